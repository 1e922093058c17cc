"""Long sequences (N = 32768 and 65536) on the GPU, beyond the BASELINE
configurations' N <= 8192: the kernels' row and tile indexing over many more
query and key tiles, GQA, causal and dense, both head-dim families.

The float64 oracle needs O(N^2 D) work per head in numpy, minutes at these
sizes, so the bar is a float32 torch restatement on the GPU (plain matmuls in
chunks of query rows, the same formulas as test_gpu_configs.fp32_reference)
with the fp16 bars of helpers.py; the oracle pins the same code paths at small
sizes (test_gpu_parity.py). The gradients' max-type bar is taken per block of
positions (rel_rms_blocks below says why).
"""
import math

import pytest
import torch

from helpers import FWD_MAX_ABS, GRAD_REL_L2, REF_REL, make_inputs

pytestmark = pytest.mark.gpu

CASES = {
    "N32768 D128 GQA causal": dict(B=1, Hq=2, Hkv=1, N=32768, D=128, causal=True),
    "N32768 D64 dense": dict(B=1, Hq=1, Hkv=1, N=32768, D=64, causal=False),
    "N65536 D64 causal": dict(B=1, Hq=1, Hkv=1, N=65536, D=64, causal=True),
    "N65536 D128 causal": dict(B=1, Hq=1, Hkv=1, N=65536, D=128, causal=True),
}
ROWS = 2048  # query rows per chunk of the reference


def fp32_reference_chunked(q, k, v, do, causal):
    """O, dQ, dK, dV in float32, one query head and ROWS query rows at a time
    (a chunk's scores against the keys it may see: at most ROWS x N floats)."""
    B, Hq, N, D = q.shape
    G = Hq // k.shape[1]
    scale = 1.0 / math.sqrt(D)
    o = torch.empty(q.shape, device=q.device)
    dq = torch.empty(q.shape, device=q.device)
    dk = torch.zeros(k.shape, device=q.device)
    dv = torch.zeros(k.shape, device=q.device)
    for b in range(B):
        for h in range(Hq):
            kh, vh = k[b, h // G].float(), v[b, h // G].float()
            for r0 in range(0, N, ROWS):
                r1 = min(N, r0 + ROWS)
                kend = r1 if causal else N
                qc, doc = q[b, h, r0:r1].float(), do[b, h, r0:r1].float()
                kc, vc = kh[:kend], vh[:kend]
                s = (qc @ kc.t().contiguous()) * scale
                if causal:
                    rows = torch.arange(r0, r1, device=q.device)[:, None]
                    cols = torch.arange(kend, device=q.device)[None, :]
                    s.masked_fill_(cols > rows, float("-inf"))
                p = torch.softmax(s, -1)
                del s
                oc = p @ vc
                dvec = (doc * oc).sum(-1, keepdim=True)
                ds = p * (doc @ vc.t().contiguous() - dvec)
                o[b, h, r0:r1] = oc
                dq[b, h, r0:r1] = (ds @ kc) * scale
                dk[b, h // G, :kend] += (ds.t().contiguous() @ qc) * scale
                dv[b, h // G, :kend] += p.t().contiguous() @ doc
                del p, ds
    return o, dq, dk, dv


def rel_l2(a, b):
    return ((a.float() - b).norm() / b.norm()).item()


def rel_rms(a, b):
    return ((a.float() - b).abs().max() / b.pow(2).mean().sqrt()).item()


def rel_rms_blocks(a, b, block=2048):
    """The reference's max|err| / RMS(ref), per block of `block` sequence
    positions (dim 2), worst block."""
    worst = 0.0
    for p0 in range(0, b.shape[2], block):
        worst = max(worst, rel_rms(a[:, :, p0:p0 + block], b[:, :, p0:p0 + block]))
    return worst


# The gradients' max-type bar is the reference's max|err| / RMS(ref) < 6e-2,
# taken per block of 2048 sequence positions. Under causal masking at these
# lengths the gradients' magnitudes fall with position by orders of magnitude
# (key 0 sums over every query row, the last key over one), so over the whole
# tensor the bar would measure the fp16 rounding of the largest entries
# against an RMS set by the many small ones (at N = 65536, D = 128: 0.071 for
# dV, from rounding alone); within a block the magnitudes are comparable.


@pytest.mark.parametrize("name", list(CASES))
def test_long_sequence_matches_fp32_reference(name):
    import fa_p100
    c = CASES[name]
    print(name, flush=True)
    q, k, v, do = make_inputs(c["B"], c["Hq"], c["Hkv"], c["N"], c["D"], seed=3)
    qg, kg, vg = (t.cuda().requires_grad_(True) for t in (q, k, v))
    dog = do.cuda()
    o = fa_p100.flash_attn(qg, kg, vg, c["causal"])
    o.backward(dog)
    torch.cuda.synchronize()
    ro, rdq, rdk, rdv = fp32_reference_chunked(qg.detach(), kg.detach(), vg.detach(), dog,
                                               c["causal"])
    err = (o.float() - ro).abs().max().item()
    assert err <= FWD_MAX_ABS, f"{name} fwd max-abs {err:.3e}"
    assert rel_rms(o, ro) < REF_REL, f"{name} fwd rel {rel_rms(o, ro):.3e}"
    for g, r, n in ((qg.grad, rdq, "dQ"), (kg.grad, rdk, "dK"), (vg.grad, rdv, "dV")):
        assert torch.isfinite(g).all(), f"{name} {n} non-finite"
        l2 = rel_l2(g, r)
        assert l2 <= GRAD_REL_L2, f"{name} {n} rel-L2 {l2:.3e}"
        rb = rel_rms_blocks(g, r)
        assert rb < REF_REL, f"{name} {n} rel per block {rb:.3e}"
