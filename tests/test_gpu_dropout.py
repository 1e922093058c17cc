"""Attention dropout (beyond the reference, whose hook raises on it,
fa_p100_hf.py:83-85): flash_attn(..., dropout_p=p, dropout_seed=s).

The keep bits come from one HIP kernel (fa_dropout_bits); here they are
checked bit for bit against the oracle's restatement of the draw
(oracle.attention.dropout_keep, pinned in test_oracle.py by plain integer
arithmetic, hand-computed entries and its statistics) in both layouts.
Forward, LSE and gradients then match the float64 oracle with the same keep
mask (its dropout forward and backward pinned against torch autograd and
finite differences), with other options too; runs repeat bit for bit under
one seed; the (B, N, H, D) views and the C ABI are bit-identical to the op;
and Qwen3 with attention dropout trains through the hook. Bars: the fp16
ones (helpers.py), bf16's from test_gpu_bf16.py."""
import ctypes

import numpy as np
import pytest
import torch

from helpers import (FWD_MAX_ABS, GRAD_REL_L2, LSE_MAX_ABS, REF_REL, fa_opts, load_capi,
                     make_inputs, np64)
from oracle import attention as ora
from test_gpu_mask import as_u32, host_words

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.mark.parametrize("p", [0.0, 0.1, 0.5, 0.9])
@pytest.mark.parametrize("planes,N", [(1, 1), (3, 31), (2, 33), (2, 64), (1, 100), (4, 1000)])
def test_dropout_bits_match_the_oracle_draw(planes, N, p):
    import fa_p100
    for seed in (0, 12345, (1 << 64) - 3):  # the last passes through a negative int64
        bits, bits_t, scale = fa_p100.dropout_bits(seed, p, 1, planes, N, DEV)
        keep, zs = ora.dropout_keep(seed, p, planes, N)
        assert bits.shape == bits_t.shape == (1, planes, N, (N + 31) // 32)
        assert np.array_equal(as_u32(bits[0]), host_words(keep)), (seed, p)
        assert np.array_equal(as_u32(bits_t[0]), host_words(np.swapaxes(keep, -1, -2)))
        assert abs(scale - zs) <= 1e-6 * zs


def test_dropout_bits_match_the_oracle_draw_on_long_rows():
    """N = 4096 (128 words per row, 16 of the generator's 8-word chunks) and
    N = 4095 (a partial last word), both layouts bit for bit."""
    import fa_p100
    for planes, n, seed in ((2, 4096, 77), (1, 4095, (1 << 63) + 5)):
        bits, bits_t, _ = fa_p100.dropout_bits(seed, 0.1, 1, planes, n, DEV)
        keep, _ = ora.dropout_keep(seed, 0.1, planes, n)
        assert np.array_equal(as_u32(bits[0]), host_words(keep)), (planes, n)
        assert np.array_equal(as_u32(bits_t[0]), host_words(np.swapaxes(keep, -1, -2))), (planes, n)


@pytest.mark.parametrize("planes,N", [(1, 1), (3, 31), (2, 33), (1, 100), (4, 1000), (1, 4095),
                                      (2, 4096)])
def test_causal_dropout_bits_match_the_oracle_draw(planes, N):
    """fa_dropout_bits_causal (what causal flash_attn draws): the full draw
    with the bits of keys j > i cleared, both layouts bit for bit, from one
    word per row to 128, ragged last words, and rows on both sides of the
    draw's 64-row waves; the forward's draw without the transpose gives the
    same words."""
    import fa_p100
    tril = np.tril(np.ones((N, N), dtype=bool))
    for seed, p in ((3, 0.1), ((1 << 64) - 9, 0.5)):
        bits, bits_t, _ = fa_p100.dropout_bits(seed, p, 1, planes, N, DEV, causal=True)
        keep, _ = ora.dropout_keep(seed, p, planes, N, causal=True)
        full, _ = ora.dropout_keep(seed, p, planes, N)
        assert not (keep & ~tril).any() and np.array_equal(keep, full & tril)
        assert np.array_equal(as_u32(bits[0]), host_words(keep)), (planes, N, seed)
        assert np.array_equal(as_u32(bits_t[0]), host_words(np.swapaxes(keep, -1, -2)))
        fwd_only, none, _ = fa_p100.dropout_bits(seed, p, 1, planes, N, DEV, transposed=False,
                                                 causal=True)
        assert none is None and torch.equal(fwd_only, bits)


@pytest.mark.parametrize("B,Hq,Hkv,N,D", [(1, 8, 8, 4096, 128), (2, 4, 2, 1000, 64)])
def test_causal_draw_leaves_causal_attention_bit_identical(B, Hq, Hkv, N, D):
    """Causal attention reads no bit of a key past the diagonal, so the
    forward and backward through the C ABI give bit-identical O, LSE, dQ, dK
    and dV with fa_dropout_bits_causal's planes and with fa_dropout_bits'
    (the headline shape and a ragged GQA one)."""
    lib = load_capi()
    q, k, v, do = (t.to(DEV) for t in make_inputs(B, Hq, Hkv, N, D, seed=N + D))
    ptr = lambda t: ctypes.c_void_p(t.data_ptr())
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    W = (N + 31) // 32
    p = 0.1
    scale = lib.fa_dropout_scale(p)
    ws_bytes = lib.fa_bwd_workspace_bytes(B, Hq, Hkv, N, D)
    ws = torch.empty(ws_bytes, device=DEV, dtype=torch.uint8)
    outs = []
    for draw in (lib.fa_dropout_bits, lib.fa_dropout_bits_causal):
        z = torch.empty(B, Hq, N, W, dtype=torch.int32, device=DEV)
        z_t = torch.empty_like(z)
        assert draw(99, p, B * Hq, N, ptr(z), ptr(z_t), s) == 0
        opts = fa_opts(drop=z, drop_t=z_t, drop_scale=scale)
        o, lse = torch.empty_like(q), torch.empty(B, Hq, N, device=DEV)
        assert lib.fa_fwd_ex(ptr(q), ptr(k), ptr(v), ptr(o), ptr(lse), B, Hq, Hkv, N, D, 1, opts,
                             s) == 0
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        rc = lib.fa_bwd_ex(ptr(q), ptr(k), ptr(v), ptr(do), ptr(o), ptr(lse), ptr(dq), ptr(dk),
                           ptr(dv), ptr(ws), ws_bytes, B, Hq, Hkv, N, D, 1, opts, s)
        assert rc == 0, lib.fa_error_string(rc)
        torch.cuda.synchronize()
        outs.append((o, lse, dq, dk, dv))
    for name, a, b in zip(("O", "LSE", "dQ", "dK", "dV"), *outs):
        assert torch.equal(a, b), name
    assert (outs[0][2] != 0).any()


def run(q, k, v, do, causal, p, seed, **kw):
    import fa_p100
    qg, kg, vg = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    o = fa_p100.flash_attn(qg, kg, vg, causal, dropout_p=p, dropout_seed=seed, **kw)
    o.backward(do.to(DEV))
    torch.cuda.synchronize()
    return o, qg.grad, kg.grad, vg.grad


def lse_of(q, k, v, causal, **kw):
    """The LSE, which dropout does not change."""
    import fa_p100
    o, lse = fa_p100._ext.forward_dt(q.to(DEV), k.to(DEV), v.to(DEV), causal, **kw)
    return lse


def check(got, lse, q, k, v, do, causal, p, seed, what, **opts):
    o, dq, dk, dv = got
    keep, zs = ora.dropout_keep(seed, p, q.shape[0] * q.shape[1], q.shape[2])
    qn, kn, vn, dn = (t.float().numpy() for t in (q, k, v, do))
    ref_o, ref_lse = ora.attention_fwd(qn, kn, vn, causal, dropout=(keep, zs), **opts)
    assert ora.max_abs(np64(o), ref_o) <= FWD_MAX_ABS * zs, what
    assert ora.rel_max_rms(np64(o), ref_o) < REF_REL, what
    seen = np.isfinite(ref_lse)
    assert ora.max_abs(np64(lse)[seen], ref_lse[seen]) <= LSE_MAX_ABS, what
    ref = ora.attention_bwd(qn, kn, vn, dn, causal, dropout=(keep, zs), **opts)
    for name, g, r in zip(("dQ", "dK", "dV"), (dq, dk, dv), ref):
        g = np64(g)
        assert np.isfinite(g).all(), (what, name)
        l2, rr = ora.rel_l2(g, r), ora.rel_max_rms(g, r)
        assert l2 <= GRAD_REL_L2 and rr < REF_REL, (what, name, l2, rr)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("D", [64, 96, 128])
@pytest.mark.parametrize("B,Hq,Hkv,N,p", [(2, 4, 2, 333, 0.1), (1, 4, 4, 1024, 0.5),
                                          (1, 2, 1, 2048, 0.2)])
def test_dropout_matches_oracle(B, Hq, Hkv, N, p, D, causal):
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, seed=N + D + causal)
    seed = 1000 + N + D
    got = run(q, k, v, do, causal, p, seed)
    check(got, lse_of(q, k, v, causal), q, k, v, do, causal, p, seed,
          f"dropout p={p} {B},{Hq}/{Hkv},N{N} D{D} causal={causal}")


@pytest.mark.parametrize("causal", [True, False])
def test_dropout_with_every_other_option(causal):
    """Dropout on top of a mask, key lengths, ALiBi and a softmax scale (and
    a window when causal)."""
    import fa_p100
    B, Hq, Hkv, N, D, p, seed = 2, 4, 2, 517, 64, 0.3, 77
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, seed=5 + causal)
    rng = np.random.default_rng(9)
    mask = rng.random((B, 1, N, N)) < 0.7
    lens = [517, 300]
    slopes = np.array([2.0 ** (-8.0 * (h + 1) / Hq) for h in range(Hq)])
    m = torch.tensor(mask, device=DEV)
    kw = dict(kv_len=torch.tensor(lens, dtype=torch.int32, device=DEV),
              alibi_slopes=torch.tensor(slopes, dtype=torch.float32, device=DEV),
              softmax_scale=0.11, attn_mask=m)
    opts = dict(kv_len=lens, alibi=np.float32(slopes).astype(np.float64),
                scale=np.float32(0.11).item(), mask=mask)
    window = 0
    if causal:
        window = 120
        kw["sliding_window"] = window
        opts["window"] = window
    got = run(q, k, v, do, causal, p, seed, **kw)
    bits, _ = fa_p100.pack_mask(m, B, Hq)
    lse = lse_of(q, k, v, causal, kv_len=kw["kv_len"], window=window,
                 alibi_slopes=kw["alibi_slopes"], scale=0.11, mask=bits)
    check(got, lse, q, k, v, do, causal, p, seed, f"dropout+options causal={causal}", **opts)


def test_dropout_repeats_bnhd_bf16_and_capi():
    """One seed gives bit-identical runs and another seed other results;
    without a seed the draw follows torch.manual_seed; the (B, N, H, D)
    views are bit-identical to the dense op; bf16 against the oracle; the C
    ABI (fa_dropout_bits, fa_fwd_ex / fa_bwd_ex with drop, drop_t,
    drop_scale) bit-identical to the op, and a backward without drop_t is
    rejected."""
    import fa_p100
    from test_gpu_bf16 import BF_FWD_MAX_ABS, BF_GRAD_REL_L2, bf16_inputs
    B, Hq, Hkv, N, D, p = 2, 8, 2, 450, 128, 0.15
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, seed=3)
    a = run(q, k, v, do, True, p, 41)
    b = run(q, k, v, do, True, p, 41)
    c = run(q, k, v, do, True, p, 42)
    for x, y in zip(a, b):
        assert torch.equal(x, y)
    assert not torch.equal(a[0], c[0])
    torch.manual_seed(7)
    d1 = run(q, k, v, do, True, p, None)
    torch.manual_seed(7)
    d2 = run(q, k, v, do, True, p, None)
    assert torch.equal(d1[0], d2[0]) and torch.equal(d1[1], d2[1])

    qb, kb, vb, gb = (t.to(DEV) for t in bf16_inputs(B, Hq, Hkv, N, D, seed=23))
    as_bnhd = lambda t: t.transpose(1, 2).contiguous().transpose(1, 2)
    dense = [t.clone().requires_grad_(True) for t in (qb, kb, vb)]
    views = [as_bnhd(t).detach().requires_grad_(True) for t in (qb, kb, vb)]
    o1 = fa_p100.flash_attn(*dense, True, dropout_p=p, dropout_seed=5)
    o2 = fa_p100.flash_attn(*views, True, dropout_p=p, dropout_seed=5)
    o1.backward(gb)
    o2.backward(as_bnhd(gb))
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)
    for x, y in zip(dense, views):
        assert torch.equal(x.grad, y.grad)
    keep, zs = ora.dropout_keep(5, p, B * Hq, N)
    f = lambda t: t.detach().float().cpu().double().numpy()
    ref_o, _ = ora.attention_fwd(f(qb), f(kb), f(vb), True, dropout=(keep, zs))
    assert ora.max_abs(f(o1), ref_o) <= BF_FWD_MAX_ABS * zs
    ref = ora.attention_bwd(f(qb), f(kb), f(vb), f(gb), True, dropout=(keep, zs))
    for t, r in zip(dense, ref):
        assert ora.rel_l2(f(t.grad), r) <= BF_GRAD_REL_L2

    lib = load_capi()
    ptr = lambda t: ctypes.c_void_p(t.data_ptr())
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    W = (N + 31) // 32
    z = torch.empty(B, Hq, N, W, dtype=torch.int32, device=DEV)
    z_t = torch.empty_like(z)
    assert lib.fa_dropout_bits(5, p, B * Hq, N, ptr(z), ptr(z_t), s) == 0
    scale = lib.fa_dropout_scale(p)
    opts = fa_opts(dtype=1, drop=z, drop_t=z_t, drop_scale=scale)
    o, lse = torch.empty_like(qb), torch.empty(B, Hq, N, device=DEV)
    assert lib.fa_fwd_ex(ptr(qb), ptr(kb), ptr(vb), ptr(o), ptr(lse), B, Hq, Hkv, N, D, 1, opts,
                         s) == 0
    ws_bytes = lib.fa_bwd_workspace_bytes(B, Hq, Hkv, N, D)
    ws = torch.empty(ws_bytes, device=DEV, dtype=torch.uint8)
    dq, dk, dv = torch.empty_like(qb), torch.empty_like(kb), torch.empty_like(vb)
    rc = lib.fa_bwd_ex(ptr(qb), ptr(kb), ptr(vb), ptr(gb), ptr(o), ptr(lse), ptr(dq), ptr(dk),
                       ptr(dv), ptr(ws), ws_bytes, B, Hq, Hkv, N, D, 1, opts, s)
    assert rc == 0, lib.fa_error_string(rc)
    torch.cuda.synchronize()
    assert torch.equal(o, o1)
    for got, t in zip((dq, dk, dv), dense):
        assert torch.equal(got, t.grad)
    no_t = fa_opts(dtype=1, drop=z, drop_scale=scale)
    assert lib.fa_bwd_ex(ptr(qb), ptr(kb), ptr(vb), ptr(gb), ptr(o), ptr(lse), ptr(dq), ptr(dk),
                         ptr(dv), ptr(ws), ws_bytes, B, Hq, Hkv, N, D, 1, no_t, s) == 10015


def test_hf_hook_trains_with_attention_dropout():
    """Qwen3 with attention_dropout 0.1 through the hook: in training the
    attention output follows the dropout (other logits than without it,
    repeated exactly under one torch seed, finite loss and gradients); in
    eval mode transformers passes no dropout, and the logits equal those of
    the same weights with attention_dropout 0."""
    import fa_p100_hf
    from transformers import Qwen3Config, Qwen3ForCausalLM

    def model_with(dropout):
        cfg = Qwen3Config(vocab_size=1000, hidden_size=512, intermediate_size=1024,
                          num_hidden_layers=2, num_attention_heads=8, num_key_value_heads=2,
                          head_dim=64, max_position_embeddings=1024, use_cache=False,
                          attention_dropout=dropout)
        torch.manual_seed(0)
        with torch.device(DEV):
            m = Qwen3ForCausalLM(cfg)
        fa_p100_hf.enable_fa_p100(m)
        return m

    ids = torch.randint(0, 1000, (2, 300), device=DEV, generator=torch.Generator(DEV).manual_seed(3))
    drop, plain = model_with(0.1), model_with(0.0)

    def train_loss(m, seed):
        m.train()
        m.zero_grad(set_to_none=True)
        torch.manual_seed(seed)
        with torch.autocast("cuda", torch.float16):
            out = m(ids, labels=ids)
        out.loss.backward()
        grads = [p.grad.float().clone() for p in m.parameters() if p.grad is not None]
        return out.logits.float().detach(), out.loss.item(), grads

    l1, loss1, g1 = train_loss(drop, 11)
    l2, loss2, g2 = train_loss(drop, 11)
    l0, loss0, _ = train_loss(plain, 11)
    assert torch.equal(l1, l2) and loss1 == loss2
    assert all(torch.equal(a, b) for a, b in zip(g1, g2))
    assert np.isfinite(loss1) and all(torch.isfinite(g).all() for g in g1)
    assert not torch.equal(l1, l0)
    drop.eval()
    plain.eval()
    with torch.no_grad(), torch.autocast("cuda", torch.float16):
        assert torch.equal(drop(ids).logits, plain(ids).logits)
