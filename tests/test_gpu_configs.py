"""The BASELINE configurations at full size, on the GPU.

Inputs follow BASELINE.md: q, k, v, dO drawn in that order from one CPU
torch.Generator().manual_seed(0) as N(0,1) (x0.5 for C4), cast to fp16. At
these sizes the float64 CPU oracle is slow, so the comparison is against a
float32 torch restatement on the GPU (plain matmuls, per query head), which
is the "fp32 math on the same seeded inputs" the tolerances are stated for.
The float64 oracle covers the same code paths at small sizes
(test_gpu_parity.py); here one head of each config is additionally checked
against it.
"""
import math

import numpy as np
import pytest
import torch

from helpers import FWD_MAX_ABS, GRAD_REL_L2, REF_REL, make_inputs, np64
from oracle import attention as ora

pytestmark = pytest.mark.gpu

CONFIGS = {
    "C2": dict(B=1, Hq=16, Hkv=16, N=2048, D=64, causal=True, s=1.0),
    "C3": dict(B=1, Hq=8, Hkv=8, N=4096, D=128, causal=True, s=1.0),
    "C4": dict(B=2, Hq=32, Hkv=8, N=3001, D=128, causal=False, s=0.5),
    # The metric's D=64 leg and a C5 layer's attention: grids of two or more
    # workgroups per CU, which the forward runs as two 4-wave workgroups per
    # CU (C2 and C3 run its 8-wave shape, C4 the 4-wave one), and the
    # backward too at width 64 (D64, W4C64).
    "D64": dict(B=1, Hq=16, Hkv=16, N=4096, D=64, causal=True, s=1.0),
    "C5L": dict(B=1, Hq=16, Hkv=8, N=8192, D=128, causal=True, s=1.0),
    # N a multiple of that shape's 64-key stage but not of the 8-wave shape's
    # 128: the two-workgroup forward's unmasked copy serves them.
    "W4C64": dict(B=1, Hq=16, Hkv=16, N=4160, D=64, causal=True, s=1.0),
    "W4D128": dict(B=1, Hq=8, Hkv=4, N=4160, D=128, causal=False, s=1.0),
}


def fp32_reference(q, k, v, do, causal):
    """O, dQ, dK, dV in float32 on the GPU, one query head at a time."""
    B, Hq, N, D = q.shape
    G = Hq // k.shape[1]
    scale = 1.0 / math.sqrt(D)
    o = torch.empty(q.shape, device=q.device)
    dq = torch.empty(q.shape, device=q.device)
    dk = torch.zeros(k.shape, device=q.device)
    dv = torch.zeros(k.shape, device=q.device)
    mask = torch.triu(torch.ones(N, N, dtype=torch.bool, device=q.device), 1) if causal else None
    for b in range(B):
        for h in range(Hq):
            qh, doh = q[b, h].float(), do[b, h].float()
            kh, vh = k[b, h // G].float(), v[b, h // G].float()
            s = (qh @ kh.t().contiguous()) * scale
            if causal:
                s.masked_fill_(mask, float("-inf"))
            p = torch.softmax(s, -1)
            oh = p @ vh
            dvec = (doh * oh).sum(-1, keepdim=True)
            ds = p * (doh @ vh.t().contiguous() - dvec)
            o[b, h] = oh
            dq[b, h] = (ds @ kh) * scale
            dk[b, h // G] += (ds.t().contiguous() @ qh) * scale
            dv[b, h // G] += p.t().contiguous() @ doh
    return o, dq, dk, dv


def rel_l2(a, b):
    return ((a.float() - b).norm() / b.norm()).item()


def rel_rms(a, b):
    return ((a.float() - b).abs().max() / b.pow(2).mean().sqrt()).item()


@pytest.mark.parametrize("name", list(CONFIGS))
def test_baseline_config(name):
    import fa_p100
    c = CONFIGS[name]
    q, k, v, do = make_inputs(c["B"], c["Hq"], c["Hkv"], c["N"], c["D"], seed=0,
                              scale_qk=c["s"], scale_vg=c["s"])
    qg, kg, vg = (t.cuda().requires_grad_(True) for t in (q, k, v))
    dog = do.cuda()
    o = fa_p100.flash_attn(qg, kg, vg, c["causal"])
    o.backward(dog)
    ro, rdq, rdk, rdv = fp32_reference(qg.detach(), kg.detach(), vg.detach(), dog, c["causal"])
    err = (o.float() - ro).abs().max().item()
    assert err <= FWD_MAX_ABS, f"{name} fwd max-abs {err:.3e}"
    assert rel_rms(o, ro) < REF_REL
    for g, r, n in ((qg.grad, rdq, "dQ"), (kg.grad, rdk, "dK"), (vg.grad, rdv, "dV")):
        assert torch.isfinite(g).all(), f"{name} {n} non-finite"
        l2 = rel_l2(g, r)
        assert l2 <= GRAD_REL_L2, f"{name} {n} rel-L2 {l2:.3e}"
        assert rel_rms(g, r) < REF_REL, f"{name} {n} rel {rel_rms(g, r):.3e}"

    # One query head (and its kv head) against the float64 oracle (up to
    # N = 4096: at 8192 its float64 N x N planes take most of a minute).
    if c["N"] > 4096:
        return
    G = c["Hq"] // c["Hkv"]
    h = c["Hq"] - 1
    hk = h // G
    qs, dos = q[:1, h:h + 1].numpy(), do[:1, h:h + 1].numpy()
    ks, vs = k[:1, hk:hk + 1].numpy(), v[:1, hk:hk + 1].numpy()
    ref_o, _ = ora.attention_fwd(qs, ks, vs, c["causal"])
    assert ora.max_abs(np64(o[:1, h:h + 1]), ref_o) <= FWD_MAX_ABS
    dq64, _, _ = ora.attention_bwd(qs, ks, vs, dos, c["causal"])
    assert ora.rel_l2(np64(qg.grad[:1, h:h + 1]), dq64) <= GRAD_REL_L2


@pytest.mark.parametrize("D, causal", [(64, True), (128, False)])
def test_two_workgroup_forward_bf16_and_bnhd(D, causal):
    """The forward's two-workgroup shape (a grid of at least two workgroups
    per CU) in bf16 against the fp32 restatement, and on (B, N, H, D)-stored
    views bit-identical to dense tensors."""
    import fa_p100
    from test_gpu_bf16 import BF_FWD_MAX_ABS, BF_GRAD_REL_L2, bf16_inputs
    B, Hq, Hkv, N = 1, 16, 8, 4096
    q, k, v, do = (t.cuda() for t in bf16_inputs(B, Hq, Hkv, N, D, seed=23))
    as_bnhd = lambda t: t.transpose(1, 2).contiguous().transpose(1, 2)
    dense = [t.clone().requires_grad_(True) for t in (q, k, v)]
    views = [as_bnhd(t).detach().requires_grad_(True) for t in (q, k, v)]
    o1 = fa_p100.flash_attn(*dense, causal)
    o2 = fa_p100.flash_attn(*views, causal)
    o1.backward(do)
    o2.backward(as_bnhd(do))
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)
    for x, y in zip(dense, views):
        assert torch.equal(x.grad, y.grad)
    ro, rdq, rdk, rdv = fp32_reference(q, k, v, do, causal)
    assert (o1.float() - ro).abs().max().item() <= BF_FWD_MAX_ABS
    for g, r, n in ((dense[0].grad, rdq, "dQ"), (dense[1].grad, rdk, "dK"),
                    (dense[2].grad, rdv, "dV")):
        assert rel_l2(g, r) <= BF_GRAD_REL_L2, n


@pytest.mark.parametrize("N, causal, bf16", [(4096, False, False), (4160, False, True),
                                             (4160, True, False)])
def test_two_workgroup_backward_width_64(N, causal, bf16):
    """The backward's two-workgroup shape at width 64 (B=2, Hkv=8: 2 * 8 *
    ceil(N/128) >= 512 workgroups, two per CU): the unmasked (N = 4096) and
    masked (N = 4160) copies, dense and causal, fp16 and bf16, against the
    fp32 restatement; (B, N, H, D)-stored views bit-identical to dense
    tensors; a second run bit-identical to the first."""
    import fa_p100
    from test_gpu_bf16 import BF_FWD_MAX_ABS, BF_GRAD_REL_L2, bf16_inputs
    B, Hq, Hkv, D = 2, 16, 8, 64
    if bf16:
        q, k, v, do = (t.cuda() for t in bf16_inputs(B, Hq, Hkv, N, D, seed=31))
        fwd_bar, grad_bar = BF_FWD_MAX_ABS, BF_GRAD_REL_L2
    else:
        q, k, v, do = (t.cuda() for t in make_inputs(B, Hq, Hkv, N, D, seed=31))
        fwd_bar, grad_bar = FWD_MAX_ABS, GRAD_REL_L2
    as_bnhd = lambda t: t.transpose(1, 2).contiguous().transpose(1, 2)
    runs = []
    for make in (lambda t: t.clone(), lambda t: t.clone(), as_bnhd):
        xs = [make(t).detach().requires_grad_(True) for t in (q, k, v)]
        o = fa_p100.flash_attn(*xs, causal)
        o.backward(make(do))
        torch.cuda.synchronize()
        runs.append((o, *(x.grad for x in xs)))
    for a, b, c in zip(*runs):
        assert torch.equal(a, b) and torch.equal(a, c)
    ro, rdq, rdk, rdv = fp32_reference(q, k, v, do, causal)
    o, dq, dk, dv = runs[0]
    assert (o.float() - ro).abs().max().item() <= fwd_bar
    for g, r, n in ((dq, rdq, "dQ"), (dk, rdk, "dK"), (dv, rdv, "dV")):
        assert torch.isfinite(g).all(), n
        assert rel_l2(g, r) <= grad_bar, (n, rel_l2(g, r))
        if not bf16:
            assert rel_rms(g, r) < REF_REL, (n, rel_rms(g, r))
