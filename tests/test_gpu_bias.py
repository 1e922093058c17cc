"""Additive attention bias (beyond the reference, which has no bias input,
HANDOFF.md:281 "attention bias is second"): flash_attn(..., attn_bias=b),
b added to the scaled scores as torch SDPA adds a float attn_mask, with its
gradient when it requires one.

Checked against the float64 oracle (its bias and dS pinned in
test_oracle.py against SDPA with the same float attn_mask and autograd,
the bias's own gradient included, and finite differences): per-head,
batch-shared, head-shared and (N, N) biases with their gradients reduced
to the bias's shape; a bias beside a mask, dropout, key lengths, ALiBi and
a window; head dims 8, 40 and 96; bf16; the (B, N, H, D) views and the C
ABI bit-identical to the op; and Qwen3 through the hook with an additive 4-D mask carrying a bias
against eager and sdpa. Bars: the fp16 ones (helpers.py) for o, LSE and
every gradient, dbias included."""
import ctypes

import numpy as np
import pytest
import torch

from helpers import (FWD_MAX_ABS, GRAD_REL_L2, LSE_MAX_ABS, REF_REL, fa_opts, load_capi,
                     make_inputs, np64)
from oracle import attention as ora

pytestmark = pytest.mark.gpu

DEV = "cuda"


def run(q, k, v, do, bias, causal, **kw):
    import fa_p100
    qg, kg, vg = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    bg = bias.to(DEV).requires_grad_(True)
    o = fa_p100.flash_attn(qg, kg, vg, causal, attn_bias=bg, **kw)
    o.backward(do.to(DEV))
    torch.cuda.synchronize()
    return o, qg.grad, kg.grad, vg.grad, bg.grad


def check(got, lse, q, k, v, do, bias, causal, what, **opts):
    o, dq, dk, dv, db = got
    qn, kn, vn, dn = (t.float().numpy() for t in (q, k, v, do))
    bn = bias.double().numpy()
    b4 = bn.reshape((1,) * (4 - bn.ndim) + bn.shape) if bn.ndim < 4 else bn
    if bn.ndim == 3:
        b4 = bn[:, None]
    ref_o, ref_lse = ora.attention_fwd(qn, kn, vn, causal, bias=b4, **opts)
    assert ora.max_abs(np64(o), ref_o) <= FWD_MAX_ABS, what
    assert ora.rel_max_rms(np64(o), ref_o) < REF_REL, what
    seen = np.isfinite(ref_lse)
    assert ora.max_abs(np64(lse)[seen], ref_lse[seen]) <= LSE_MAX_ABS, what
    # The backward consumes the forward's saved state: dS (the bias gradient,
    # compared elementwise) uses the fp16-rounded o in Dv = rowsum(dO o), as
    # the kernels and the reference do (flash_bwd.cuh:65-78).
    ref = ora.attention_bwd(qn, kn, vn, dn, causal, o=np64(o), lse=np64(lse), bias=b4,
                            dbias=True, **opts)
    ds = ref[3]
    red = ds.sum(axis=tuple(a for a in (0, 1) if b4.shape[a] == 1), keepdims=True)
    ref_db = red.reshape(bn.shape)
    for name, g, r in zip(("dQ", "dK", "dV", "dbias"), (dq, dk, dv, db), ref[:3] + (ref_db,)):
        g = np64(g)
        assert g.shape == r.shape, (what, name, g.shape, r.shape)
        assert np.isfinite(g).all(), (what, name)
        l2, rr = ora.rel_l2(g, r), ora.rel_max_rms(g, r)
        assert l2 <= GRAD_REL_L2 and rr < REF_REL, (what, name, l2, rr)


def lse_of(q, k, v, causal, bias4, **kw):
    import fa_p100
    _, lse = fa_p100._ext.forward_dt(q.to(DEV), k.to(DEV), v.to(DEV), causal,
                                     bias=bias4.to(DEV).float(), **kw)
    return lse


def as4(bias, B, Hq):
    if bias.dim() == 2:
        return bias[None, None]
    if bias.dim() == 3:
        return bias[:, None]
    return bias


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("shape", ["BHNN", "1HNN", "B1NN", "NN", "BNN"])
@pytest.mark.parametrize("B,Hq,Hkv,N", [(2, 4, 2, 333), (1, 2, 1, 1000)])
def test_bias_matches_oracle(B, Hq, Hkv, N, shape, D, causal):
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, seed=N + D + causal)
    g = torch.Generator().manual_seed(N + len(shape))
    dims = {"BHNN": (B, Hq, N, N), "1HNN": (1, Hq, N, N), "B1NN": (B, 1, N, N),
            "NN": (N, N), "BNN": (B, N, N)}[shape]
    bias = torch.randn(*dims, generator=g) * 1.5
    got = run(q, k, v, do, bias, causal)
    check(got, lse_of(q, k, v, causal, as4(bias, B, Hq)), q, k, v, do, bias, causal,
          f"bias {shape} {B},{Hq}/{Hkv},N{N} D{D} causal={causal}")


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("D", [8, 40, 96])
def test_bias_other_head_dims(D, causal):
    """Head dims on the widths 32, 64 and 96 (columns past the head dim
    are padding in the staged Q, K and V tiles), GQA, a ragged N."""
    B, Hq, Hkv, N = 2, 4, 2, 301
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, seed=D + causal)
    bias = torch.randn(B, 1, N, N, generator=torch.Generator().manual_seed(D)) * 1.5
    got = run(q, k, v, do, bias, causal)
    check(got, lse_of(q, k, v, causal, bias), q, k, v, do, bias, causal,
          f"bias D{D} causal={causal}")


@pytest.mark.parametrize("causal", [True, False])
def test_bias_with_every_other_option(causal):
    """A bias with a mask, dropout, key lengths, ALiBi and a scale (and a
    window when causal)."""
    import fa_p100
    B, Hq, Hkv, N, D = 2, 4, 2, 517, 64
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, seed=31 + causal)
    g = torch.Generator().manual_seed(5)
    bias = torch.randn(B, Hq, N, N, generator=g)
    rng = np.random.default_rng(2)
    mask = rng.random((B, 1, N, N)) < 0.7
    lens = [517, 333]
    slopes = np.array([2.0 ** (-8.0 * (h + 1) / Hq) for h in range(Hq)])
    p, seed = 0.2, 99
    m = torch.tensor(mask, device=DEV)
    kw = dict(kv_len=torch.tensor(lens, dtype=torch.int32, device=DEV),
              alibi_slopes=torch.tensor(slopes, dtype=torch.float32, device=DEV),
              softmax_scale=0.13, attn_mask=m, dropout_p=p, dropout_seed=seed)
    opts = dict(kv_len=lens, alibi=np.float32(slopes).astype(np.float64),
                scale=np.float32(0.13).item(), mask=mask,
                dropout=ora.dropout_keep(seed, p, B * Hq, N))
    window = 0
    if causal:
        window = 140
        kw["sliding_window"] = window
        opts["window"] = window
    got = run(q, k, v, do, bias, causal, **kw)
    bits, _ = fa_p100.pack_mask(m, B, Hq)
    lse = lse_of(q, k, v, causal, bias, kv_len=kw["kv_len"], window=window,
                 alibi_slopes=kw["alibi_slopes"], scale=0.13, mask=bits)
    check(got, lse, q, k, v, do, bias, causal, f"bias+options causal={causal}", **opts)


def test_bias_bf16_bnhd_and_capi():
    """bf16 against the oracle; the (B, N, H, D) views bit-identical to the
    dense op; fa_fwd_ex / fa_bwd_ex with bias, strides and dbias
    bit-identical to the op (dbias before its reduction)."""
    import fa_p100
    from test_gpu_bf16 import BF_FWD_MAX_ABS, BF_GRAD_REL_L2, bf16_inputs
    B, Hq, Hkv, N, D = 2, 8, 2, 450, 128
    q, k, v, do = (t.to(DEV) for t in bf16_inputs(B, Hq, Hkv, N, D, seed=29))
    g = torch.Generator().manual_seed(1)
    bias = (torch.randn(1, Hq, N, N, generator=g) * 2).to(DEV)
    as_bnhd = lambda t: t.transpose(1, 2).contiguous().transpose(1, 2)
    dense = [t.clone().requires_grad_(True) for t in (q, k, v)]
    views = [as_bnhd(t).detach().requires_grad_(True) for t in (q, k, v)]
    b1, b2 = bias.clone().requires_grad_(True), bias.clone().requires_grad_(True)
    o1 = fa_p100.flash_attn(*dense, True, attn_bias=b1)
    o2 = fa_p100.flash_attn(*views, True, attn_bias=b2)
    o1.backward(do)
    o2.backward(as_bnhd(do))
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(b1.grad, b2.grad)
    for a, b in zip(dense, views):
        assert torch.equal(a.grad, b.grad)
    f = lambda t: t.detach().float().cpu().double().numpy()
    ref_o, _ = ora.attention_fwd(f(q), f(k), f(v), True, bias=f(bias))
    assert ora.max_abs(f(o1), ref_o) <= BF_FWD_MAX_ABS
    ref = ora.attention_bwd(f(q), f(k), f(v), f(do), True, bias=f(bias), dbias=True)
    for t, r in zip(dense, ref[:3]):
        assert ora.rel_l2(f(t.grad), r) <= BF_GRAD_REL_L2
    assert ora.rel_l2(f(b1.grad), ref[3].sum(axis=0, keepdims=True)) <= BF_GRAD_REL_L2

    lib = load_capi()
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    dbias = torch.zeros(B, Hq, N, N, device=DEV)
    opts = fa_opts(dtype=1, bias=bias, bias_stride_b=0, bias_stride_h=N * N, dbias=dbias)
    o, lse = torch.empty_like(q), torch.empty(B, Hq, N, device=DEV)
    assert lib.fa_fwd_ex(p(q), p(k), p(v), p(o), p(lse), B, Hq, Hkv, N, D, 1, opts, s) == 0
    ws_bytes = lib.fa_bwd_workspace_bytes(B, Hq, Hkv, N, D)
    ws = torch.empty(ws_bytes, device=DEV, dtype=torch.uint8)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    rc = lib.fa_bwd_ex(p(q), p(k), p(v), p(do), p(o), p(lse), p(dq), p(dk), p(dv), p(ws),
                       ws_bytes, B, Hq, Hkv, N, D, 1, opts, s)
    assert rc == 0, lib.fa_error_string(rc)
    torch.cuda.synchronize()
    assert torch.equal(o, o1)
    for got, t in zip((dq, dk, dv), dense):
        assert torch.equal(got, t.grad)
    assert torch.equal(dbias.sum(0, keepdim=True), b1.grad)


def test_hf_hook_additive_bias_mask_matches_eager():
    """Qwen3 through the hook with a 4-D additive mask that carries a bias
    (a causal mask plus a per-head distance bias, as T5-style models build
    one): logits within the eager-vs-sdpa envelope of eager with the same
    mask."""
    import fa_p100_hf
    from test_gpu_hf import qwen3
    N, H = 280, 8
    ids = torch.randint(0, 1000, (2, N), device=DEV, generator=torch.Generator(DEV).manual_seed(6))
    model = qwen3(2, 512, H, 2, 64, 1024, 1000).eval()
    i = torch.arange(N, device=DEV)[:, None]
    j = torch.arange(N, device=DEV)[None, :]
    slopes = torch.tensor([0.5 ** (h + 1) for h in range(H)], device=DEV)[:, None, None]
    bias = (-slopes * (i - j).abs().float()).masked_fill(j > i, torch.finfo(torch.float32).min)
    mask = bias[None].expand(2, H, N, N)

    def logits(impl):
        model.config._attn_implementation = impl
        with torch.no_grad(), torch.autocast("cuda", torch.float16):
            return model(ids, attention_mask=mask).logits.float()

    eager, sdpa = logits("eager"), logits("sdpa")
    fa_p100_hf.enable_fa_p100(model)
    fa = logits("fa_p100")
    env, gap = (sdpa - eager).abs(), (fa - eager).abs()
    assert gap.mean() <= 2 * env.mean() + 1e-4, (gap.mean().item(), env.mean().item())
