"""Head dims other than 64 and 128 (the reference takes those two only,
fa_p100_ext.cu:59, 111). The kernels run at the tile widths 32, 64, 96 and
128; a head dim between them runs on the next wider one, its extra columns
loaded as zeros and never stored. At width 96 (and 32) the backward's staged
tiles use padded rows (192-byte rows do not pack into the 1 KB direct
loads). The plain matrices run in test_gpu_parity.py with D=96 added. Here:
every multiple of 8 from 8 to 128 against the float64 oracle; every option
at D=96 and D=80 (key lengths, window, ALiBi, packed sequences, mask,
softmax scale); split key tiles over long causal rows; bf16, the
(B, N, H, D) views and the C ABI bit-identical to the dense op; and Qwen3
with head_dim 80 through the hook. Bars: the fp16 ones (helpers.py),
bf16's from test_gpu_bf16.py."""
import ctypes

import numpy as np
import pytest
import torch

from helpers import (FWD_MAX_ABS, GRAD_REL_L2, LSE_MAX_ABS, REF_REL, fa_opts, load_capi,
                     make_inputs, np64)
from oracle import attention as ora

pytestmark = pytest.mark.gpu

DEV = "cuda"
D = 96


def check(o, lse, grads, q, k, v, do, causal, what, **opts):
    qn, kn, vn, dn = (t.float().numpy() for t in (q, k, v, do))
    ref_o, ref_lse = ora.attention_fwd(qn, kn, vn, causal, **opts)
    assert ora.max_abs(np64(o), ref_o) <= FWD_MAX_ABS, what
    assert ora.rel_max_rms(np64(o), ref_o) < REF_REL, what
    seen = np.isfinite(ref_lse)
    assert np.array_equal(np.isfinite(np64(lse)), seen), what
    assert ora.max_abs(np64(lse)[seen], ref_lse[seen]) <= LSE_MAX_ABS, what
    ref = ora.attention_bwd(qn, kn, vn, dn, causal, **opts)
    for name, g, r in zip(("dQ", "dK", "dV"), grads, ref):
        g = np64(g)
        assert np.isfinite(g).all(), (what, name)
        l2, rr = ora.rel_l2(g, r), ora.rel_max_rms(g, r)
        assert l2 <= GRAD_REL_L2 and rr < REF_REL, (what, name, l2, rr)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("Dh", list(range(8, 129, 8)))
def test_every_head_dim_matches_oracle(Dh, causal):
    """Each multiple of 8 up to 128 on a ragged shape with GQA and two key
    tiles per workgroup (the causal split included)."""
    import fa_p100
    B, Hq, Hkv, N = 2, 4, 2, 397
    q, k, v, do = make_inputs(B, Hq, Hkv, N, Dh, seed=Dh + causal)
    qg, kg, vg = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    o = fa_p100.flash_attn(qg, kg, vg, causal)
    o.backward(do.to(DEV))
    _, lse = fa_p100._ext.forward(qg.detach(), kg.detach(), vg.detach(), causal, False)
    torch.cuda.synchronize()
    assert o.shape == q.shape and qg.grad.shape == q.shape and kg.grad.shape == k.shape
    check(o, lse, (qg.grad, kg.grad, vg.grad), q, k, v, do, causal, f"D{Dh} causal={causal}")


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("B,Hq,Hkv,N", [(1, 4, 4, 2048), (2, 8, 2, 1000), (1, 2, 1, 4096)])
def test_d96_long_rows_match_oracle(B, Hq, Hkv, N, causal):
    """Long rows: several key tiles per workgroup, the causal split of key
    tiles between workgroups (N >= 384), GQA and MQA."""
    import fa_p100
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, seed=N + Hkv + causal)
    qg, kg, vg = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    o = fa_p100.flash_attn(qg, kg, vg, causal)
    o.backward(do.to(DEV))
    _, lse = fa_p100._ext.forward(qg.detach(), kg.detach(), vg.detach(), causal, False)
    torch.cuda.synchronize()
    check(o, lse, (qg.grad, kg.grad, vg.grad), q, k, v, do, causal,
          f"D96 {B},{Hq}/{Hkv},N{N} causal={causal}")


@pytest.mark.parametrize("D", [96, 80])
@pytest.mark.parametrize("causal", [True, False])
def test_d96_every_option_matches_oracle(causal, D):
    """Key lengths, ALiBi, a softmax scale, packed sequences, a mask, and a
    window when causal, all at once."""
    import fa_p100
    B, Hq, Hkv, N = 2, 4, 2, 777
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, seed=31 + causal)
    lens = [777, 500]
    slopes = np.array([2.0 ** (-8.0 * (h + 1) / Hq) for h in range(Hq)])
    seg = np.stack([np.repeat([0, 1, 2], [300, 1, 476]), np.repeat([5, 6], [400, 377])])
    rng = np.random.default_rng(3 + causal)
    mask = rng.random((B, 1, N, N)) < 0.8
    kw = dict(kv_len=torch.tensor(lens, dtype=torch.int32, device=DEV),
              alibi_slopes=torch.tensor(slopes, dtype=torch.float32, device=DEV),
              softmax_scale=0.09, segment_ids=torch.tensor(seg, device=DEV),
              attn_mask=torch.tensor(mask, device=DEV))
    opts = dict(kv_len=lens, alibi=np.float32(slopes).astype(np.float64),
                scale=np.float32(0.09).item(), segments=seg, mask=mask)
    window = 0
    if causal:
        window = 150
        kw["sliding_window"] = window
        opts["window"] = window
    qg, kg, vg = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    o = fa_p100.flash_attn(qg, kg, vg, causal, **kw)
    o.backward(do.to(DEV))
    s0, s1 = fa_p100.segment_bounds(kw["segment_ids"])
    bits, _ = fa_p100.pack_mask(kw["attn_mask"], B, Hq)
    _, lse = fa_p100._ext.forward_dt(qg.detach(), kg.detach(), vg.detach(), causal, kw["kv_len"],
                                     window, kw["alibi_slopes"], s0, s1, 0.09, bits)
    torch.cuda.synchronize()
    check(o, lse, (qg.grad, kg.grad, vg.grad), q, k, v, do, causal,
          f"D{D} options causal={causal}", **opts)


@pytest.mark.parametrize("D", [96, 40])
def test_d96_bf16_bnhd_and_capi(D):
    """bf16 against the oracle; (B, N, H, D) views bit-identical to the dense
    op; fa_fwd / fa_bwd (fp16) and fa_fwd_ex / fa_bwd_ex (bf16) through the C
    ABI bit-identical to the op."""
    import fa_p100
    from test_gpu_bf16 import BF_FWD_MAX_ABS, BF_GRAD_REL_L2, bf16_inputs
    B, Hq, Hkv, N = 2, 8, 2, 555
    q, k, v, do = (t.to(DEV) for t in bf16_inputs(B, Hq, Hkv, N, D, seed=19))
    as_bnhd = lambda t: t.transpose(1, 2).contiguous().transpose(1, 2)
    dense = [t.clone().requires_grad_(True) for t in (q, k, v)]
    views = [as_bnhd(t).detach().requires_grad_(True) for t in (q, k, v)]
    o1 = fa_p100.flash_attn(*dense, True)
    o2 = fa_p100.flash_attn(*views, True)
    o1.backward(do)
    o2.backward(as_bnhd(do))
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)
    for a, b in zip(dense, views):
        assert torch.equal(a.grad, b.grad)
    f = lambda t: t.detach().float().cpu().double().numpy()
    ref_o, _ = ora.attention_fwd(f(q), f(k), f(v), True)
    assert ora.max_abs(f(o1), ref_o) <= BF_FWD_MAX_ABS
    ref = ora.attention_bwd(f(q), f(k), f(v), f(do), True)
    for t, r in zip(dense, ref):
        assert ora.rel_l2(f(t.grad), r) <= BF_GRAD_REL_L2

    lib = load_capi()
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    o, lse = torch.empty_like(q), torch.empty(B, Hq, N, device=DEV)
    opts = fa_opts(dtype=1)
    assert lib.fa_fwd_ex(p(q), p(k), p(v), p(o), p(lse), B, Hq, Hkv, N, D, 1, opts, s) == 0
    ws_bytes = lib.fa_bwd_workspace_bytes(B, Hq, Hkv, N, D)
    assert ws_bytes > 0
    ws = torch.empty(ws_bytes, device=DEV, dtype=torch.uint8)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    rc = lib.fa_bwd_ex(p(q), p(k), p(v), p(do), p(o), p(lse), p(dq), p(dk), p(dv), p(ws),
                       ws_bytes, B, Hq, Hkv, N, D, 1, opts, s)
    assert rc == 0, lib.fa_error_string(rc)
    torch.cuda.synchronize()
    assert torch.equal(o, o1)
    for got, t in zip((dq, dk, dv), dense):
        assert torch.equal(got, t.grad)

    # fp16 through the reference-shaped entry points: fp32 dq, as the reference.
    qh, kh, vh, gh = (t.half() for t in (q, k, v, do))
    oh, lh = torch.empty_like(qh), torch.empty(B, Hq, N, device=DEV)
    assert lib.fa_fwd(p(qh), p(kh), p(vh), p(oh), p(lh), B, Hq, Hkv, N, D, 1, 0, s) == 0
    dq32 = torch.empty(B, Hq, N, D, device=DEV)
    dkh, dvh = torch.empty_like(kh), torch.empty_like(vh)
    rc = lib.fa_bwd(p(qh), p(kh), p(vh), p(gh), p(oh), p(lh), p(dq32), p(dkh), p(dvh), p(ws),
                    ws_bytes, B, Hq, Hkv, N, D, 1, s)
    assert rc == 0, lib.fa_error_string(rc)
    torch.cuda.synchronize()
    o_ref, l_ref = fa_p100._ext.forward(qh, kh, vh, True, False)
    assert torch.equal(oh, o_ref) and torch.equal(lh, l_ref)
    dq_ref, dk_ref, dv_ref = fa_p100._ext.backward(qh, kh, vh, gh, oh, lh, True)
    assert torch.equal(dq32, dq_ref) and torch.equal(dkh, dk_ref) and torch.equal(dvh, dv_ref)


def test_hf_hook_head_dim_80_matches_eager():
    """Qwen3 with head_dim 80 (a width between the tiles) through the hook:
    logits within the eager-vs-sdpa envelope."""
    import fa_p100_hf
    from test_gpu_hf import logits_with, qwen3
    model = qwen3(2, 640, 8, 4, 80, 1024, 1000).eval()
    ids = torch.randint(0, 1000, (2, 300), device=DEV, generator=torch.Generator(DEV).manual_seed(2))
    eager, sdpa = logits_with(model, "eager", ids), logits_with(model, "sdpa", ids)
    fa_p100_hf.enable_fa_p100(model)
    fa = logits_with(model, "fa_p100", ids)
    env, gap = (sdpa - eager).abs(), (fa - eager).abs()
    assert gap.mean() <= 2 * env.mean() + 1e-4, (gap.mean().item(), env.mean().item())
