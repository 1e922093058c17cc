"""Very large grids on the GPU: B*Hq = 65536 and more (query heads or batch
entries), where every launch's 1-D grid holds tens of thousands of
workgroups (the shape limits are checked on the CPU in test_boundary_cpu.py).

At these sizes each head is short, so the bar is a float32 torch
restatement on the GPU, batched over heads (torch.bmm on contiguous
operands), with the fp16 bars of helpers.py.
"""
import math

import pytest
import torch

from helpers import FWD_MAX_ABS, GRAD_REL_L2, REF_REL

pytestmark = pytest.mark.gpu

CASES = {
    "65536 heads N64 D64 causal": dict(B=1, Hq=65536, Hkv=65536, N=64, D=64, causal=True),
    "65536 batch entries N1 D64": dict(B=65536, Hq=1, Hkv=1, N=1, D=64, causal=True),
    "B2 32768 heads GQA N128 D128": dict(B=2, Hq=32768, Hkv=8, N=128, D=128, causal=False),
}
CHUNK = 4096  # heads per batched reference step


def fp32_reference_batched(q, k, v, do, causal):
    """O, dQ, dK, dV in float32, CHUNK (batch, query head) pairs at a time."""
    B, Hq, N, D = q.shape
    Hkv = k.shape[1]
    G = Hq // Hkv
    scale = 1.0 / math.sqrt(D)
    qf, dof = q.reshape(B * Hq, N, D), do.reshape(B * Hq, N, D)
    # Query head h reads kv head h // G (repeat_interleave, fa_p100.py:62).
    kf = k.repeat_interleave(G, dim=1).reshape(B * Hq, N, D)
    vf = v.repeat_interleave(G, dim=1).reshape(B * Hq, N, D)
    o = torch.empty(B * Hq, N, D, device=q.device)
    dq = torch.empty_like(o)
    dk = torch.empty_like(o)
    dv = torch.empty_like(o)
    mask = torch.triu(torch.ones(N, N, dtype=torch.bool, device=q.device), 1) if causal else None
    for c0 in range(0, B * Hq, CHUNK):
        sl = slice(c0, min(B * Hq, c0 + CHUNK))
        qc, kc, vc, doc = (t[sl].float() for t in (qf, kf, vf, dof))
        s = torch.bmm(qc, kc.transpose(1, 2).contiguous()) * scale
        if causal:
            s.masked_fill_(mask, float("-inf"))
        p = torch.softmax(s, -1)
        oc = torch.bmm(p, vc)
        dvec = (doc * oc).sum(-1, keepdim=True)
        ds = p * (torch.bmm(doc, vc.transpose(1, 2).contiguous()) - dvec)
        o[sl] = oc
        dq[sl] = torch.bmm(ds, kc) * scale
        dk[sl] = torch.bmm(ds.transpose(1, 2).contiguous(), qc) * scale
        dv[sl] = torch.bmm(p.transpose(1, 2).contiguous(), doc)
    shape_kv = (B, Hkv, G, N, D)
    return (o.reshape(q.shape), dq.reshape(q.shape), dk.reshape(shape_kv).sum(2),
            dv.reshape(shape_kv).sum(2))


def rel_l2(a, b):
    return ((a.float() - b).norm() / b.norm()).item()


def rel_rms(a, b):
    return ((a.float() - b).abs().max() / b.pow(2).mean().sqrt()).item()


@pytest.mark.parametrize("name", list(CASES))
def test_large_grid_matches_fp32_reference(name):
    import fa_p100
    c = CASES[name]
    print(name, flush=True)
    g = torch.Generator(device="cuda").manual_seed(11)
    B, Hq, Hkv, N, D = (c[x] for x in ("B", "Hq", "Hkv", "N", "D"))
    q, do = (torch.randn(B, Hq, N, D, generator=g, device="cuda").half() for _ in range(2))
    k, v = (torch.randn(B, Hkv, N, D, generator=g, device="cuda").half() for _ in range(2))
    qg, kg, vg = (t.clone().requires_grad_(True) for t in (q, k, v))
    o = fa_p100.flash_attn(qg, kg, vg, c["causal"])
    o.backward(do)
    torch.cuda.synchronize()
    ro, rdq, rdk, rdv = fp32_reference_batched(q, k, v, do, c["causal"])
    err = (o.float() - ro).abs().max().item()
    assert err <= FWD_MAX_ABS, f"{name} fwd max-abs {err:.3e}"
    assert rel_rms(o, ro) < REF_REL, f"{name} fwd rel {rel_rms(o, ro):.3e}"
    for gr, r, n in ((qg.grad, rdq, "dQ"), (kg.grad, rdk, "dK"), (vg.grad, rdv, "dV")):
        assert gr.shape == r.shape, (name, n)
        assert torch.isfinite(gr).all(), f"{name} {n} non-finite"
        if r.abs().max().item() <= 1e-4:
            # One key per row (N = 1): dS = P (dP - Dv) is exactly zero, and
            # both the fp32 restatement and the kernels leave only fp32
            # rounding of dP - Dv (two orders of one dot product). Wrong
            # gradients are of order one here.
            assert gr.float().abs().max().item() <= 1e-4, (name, n)
            continue
        l2 = rel_l2(gr, r)
        assert l2 <= GRAD_REL_L2, f"{name} {n} rel-L2 {l2:.3e}"
        assert rel_rms(gr, r) < REF_REL, f"{name} {n} rel {rel_rms(gr, r):.3e}"
