"""Memory just past the rows of each head is never used.

Rows past N (ragged N, the last key and query tiles) are loaded through
buffer resources that end at the head's last row and are masked in the
kernels. Here q, k, v, dO and o are views at the start of allocations whose
remaining bytes hold NaN, so the last head's rows are followed by NaN
(not by another head's finite rows): any value read past a head's end and
multiplied by a masked zero would turn the results into NaN. Forward, LSE
and gradients against the float64 oracle, fp16 and bf16, every head dim,
causal and not, with key lengths too."""
import numpy as np
import pytest
import torch

from helpers import FWD_MAX_ABS, GRAD_REL_L2, LSE_MAX_ABS, make_inputs, np64
from oracle import attention as ora

pytestmark = pytest.mark.gpu

DEV = "cuda"


def nan_tail(t, rows_after):
    """t copied to the start of a fresh allocation followed by NaN."""
    extra = rows_after * t.size(-1)
    store = torch.full((t.numel() + extra,), float("nan"), dtype=t.dtype, device=DEV)
    view = store[: t.numel()].view(t.shape)
    view.copy_(t.to(DEV))
    return view


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("D", [64, 96, 128])
@pytest.mark.parametrize("N,lens", [(333, None), (200, [200, 77]), (1, None)])
def test_rows_past_each_head_are_never_used(D, causal, dtype, N, lens):
    import fa_p100
    B, Hq, Hkv = 2, 4, 2
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, seed=N + D)
    q, k, v, do = (t.to(dtype) for t in (q, k, v, do))
    kv_len = None if lens is None else torch.tensor(lens, dtype=torch.int32, device=DEV)
    qg, kg, vg = (nan_tail(t, 256).requires_grad_(True) for t in (q, k, v))
    o = fa_p100.flash_attn(qg, kg, vg, causal, kv_len=kv_len)
    o.backward(nan_tail(do, 256))
    # The backward's own o and lse inputs followed by NaN as well.
    o2, lse = fa_p100._ext.forward_dt(qg.detach(), kg.detach(), vg.detach(), causal, kv_len)
    dq, dk, dv = fa_p100._ext.backward_dt(qg.detach(), kg.detach(), vg.detach(),
                                          nan_tail(do, 256), nan_tail(o2, 256), lse, causal,
                                          kv_len)
    torch.cuda.synchronize()
    for t in (o, qg.grad, kg.grad, vg.grad, dq, dk, dv):
        assert torch.isfinite(t).all()
    assert torch.equal(o, o2) and torch.equal(dq, qg.grad)
    assert torch.equal(dk, kg.grad) and torch.equal(dv, vg.grad)
    f = lambda t: t.detach().float().cpu().double().numpy()
    ref_o, ref_lse = ora.attention_fwd(f(q), f(k), f(v), causal, kv_len=lens)
    bar = FWD_MAX_ABS if dtype == torch.float16 else 2.5e-2
    assert ora.max_abs(f(o), ref_o) <= bar
    assert ora.max_abs(np64(lse), ref_lse) <= LSE_MAX_ABS
    ref = ora.attention_bwd(f(q), f(k), f(v), f(do), causal, kv_len=lens)
    gbar = GRAD_REL_L2 if dtype == torch.float16 else 2e-2
    for g, r in zip((dq, dk, dv), ref):
        if np.linalg.norm(r) == 0:  # N = 1: dQ = dK = 0 exactly (P = 1, so dS = 0)
            assert ora.max_abs(f(g), r) <= 1e-4
        else:
            assert ora.rel_l2(f(g), r) <= gbar
