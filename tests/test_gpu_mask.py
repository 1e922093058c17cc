"""Arbitrary boolean attention masks (beyond the reference, whose kernels take
no mask and whose hook raised on any, fa_p100_hf.py:64-70):
flash_attn(..., attn_mask=m), key j hidden from query i wherever m is False,
on top of causal masking and the other options.

Checked against the float64 oracle with the same mask (pinned in
test_oracle.py against torch SDPA's boolean attn_mask with autograd, the
masks that reduce to causal / key lengths / packed sequences, empty rows and
finite differences): per-head and head-shared masks, sparse ones that leave
rows empty (o = 0, lse = +inf), masks with key lengths, a window, ALiBi and a
softmax scale; the packer (fa_pack_mask) bit-exact against host packing; the
(B, N, H, D) views and the C ABI bit-identical to the dense op; bf16; and
Qwen3 through the hook with 2-D masks with holes and 4-D masks against eager
and sdpa with the same masks. Bars: the fp16 ones (helpers.py), bf16's from
test_gpu_bf16.py."""
import ctypes

import numpy as np
import pytest
import torch

from helpers import (FWD_MAX_ABS, GRAD_REL_L2, LSE_MAX_ABS, REF_REL, fa_opts, load_capi,
                     make_inputs, np64)
from oracle import attention as ora

pytestmark = pytest.mark.gpu

DEV = "cuda"


def host_words(dense):
    """Bits of a boolean (..., R, C) array packed on the host: bit c % 32 of
    word c // 32 of each row (little-endian bit order), as int64."""
    c = dense.shape[-1]
    w = (c + 31) // 32
    pad = np.zeros(dense.shape[:-1] + (w * 32,), dtype=bool)
    pad[..., :c] = dense
    return np.packbits(pad, axis=-1, bitorder="little").view("<u4").astype(np.int64)


def as_u32(t):
    return t.cpu().numpy().astype(np.int64) & 0xFFFFFFFF


@pytest.mark.parametrize("planes,N", [(1, 1), (3, 31), (2, 32), (2, 33), (1, 100), (3, 256),
                                      (1, 1000), (2, 4096)])
def test_pack_mask_matches_host_packing(planes, N):
    """Both layouts bit-exact against numpy's packbits, including the tail
    word (bits past N clear), on the vector path (N % 16 == 0) and the byte
    path; a base address off 16 bytes takes the byte path too."""
    import fa_p100
    rng = np.random.default_rng(planes * 7 + N)
    dense = rng.random((planes, N, N)) < 0.5
    t = torch.tensor(dense, device=DEV)
    bits, bits_t = fa_p100._ext.pack_mask(t, True)
    assert bits.shape == bits_t.shape == (planes, N, (N + 31) // 32)
    assert np.array_equal(as_u32(bits), host_words(dense))
    assert np.array_equal(as_u32(bits_t), host_words(np.swapaxes(dense, -1, -2)))
    only, = fa_p100._ext.pack_mask(t, False)
    assert torch.equal(only, bits)
    if N % 16 == 0:
        store = torch.zeros(planes * N * N + 1, dtype=torch.bool, device=DEV)
        view = store[1:].view(planes, N, N)  # contiguous, base 1 byte off
        view.copy_(t)
        b2, t2 = fa_p100._ext.pack_mask(view, True)
        assert torch.equal(b2, bits) and torch.equal(t2, bits_t)


def run(q, k, v, do, mask, causal, **kw):
    """flash_attn with the mask; o, the LSE (forward_dt with the same
    options), and the gradients."""
    import fa_p100
    m = torch.tensor(mask, device=DEV)
    qg, kg, vg = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    o = fa_p100.flash_attn(qg, kg, vg, causal, attn_mask=m, **kw)
    o.backward(do.to(DEV))
    bits, _ = fa_p100.pack_mask(m, q.size(0), q.size(1))
    kv_len = kw.get("kv_len")
    al = kw.get("alibi_slopes")
    _, lse = fa_p100._ext.forward_dt(qg.detach(), kg.detach(), vg.detach(), causal, kv_len,
                                     kw.get("sliding_window") or 0, al, None, None,
                                     kw.get("softmax_scale") or 0.0, bits)
    torch.cuda.synchronize()
    return o, lse, qg.grad, kg.grad, vg.grad


def check(got, q, k, v, do, mask, causal, what, **opts):
    o, lse, dq, dk, dv = got
    qn, kn, vn, dn = (t.float().numpy() for t in (q, k, v, do))
    ref_o, ref_lse = ora.attention_fwd(qn, kn, vn, causal, mask=mask, **opts)
    assert ora.max_abs(np64(o), ref_o) <= FWD_MAX_ABS, what
    assert ora.rel_max_rms(np64(o), ref_o) < REF_REL, what
    seen = np.isfinite(ref_lse)
    assert np.array_equal(np.isfinite(np64(lse)), seen), what
    assert ora.max_abs(np64(lse)[seen], ref_lse[seen]) <= LSE_MAX_ABS, what
    assert np.all(np64(o)[~seen] == 0), what  # rows without a key
    ref = ora.attention_bwd(qn, kn, vn, dn, causal, mask=mask, **opts)
    for name, g, r in zip(("dQ", "dK", "dV"), (dq, dk, dv), ref):
        g = np64(g)
        assert np.isfinite(g).all(), (what, name)
        l2, rr = ora.rel_l2(g, r), ora.rel_max_rms(g, r)
        assert l2 <= GRAD_REL_L2 and rr < REF_REL, (what, name, l2, rr)
    return int((~seen).sum())


def random_mask(rng, B, heads, N, density):
    return rng.random((B, heads, N, N)) < density


# (B, Hq, Hkv, N, mask heads, density): ragged and tile-aligned N, per-head
# and head-shared planes, sparse masks (rows left empty, mostly under causal
# masking) and dense ones.
CASES = [
    (2, 4, 2, 333, 4, 0.5),
    (1, 4, 1, 1000, 1, 0.05),
    (2, 2, 2, 256, 1, 0.9),
    (1, 8, 8, 130, 8, 0.3),
    (1, 2, 1, 2048, 2, 0.7),
]


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("B,Hq,Hkv,N,MH,density", CASES)
def test_mask_matches_oracle(B, Hq, Hkv, N, MH, density, D, causal):
    rng = np.random.default_rng(N + D + MH + causal)
    mask = random_mask(rng, B, MH, N, density)
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, seed=N + 3 * D + causal)
    got = run(q, k, v, do, mask, causal)
    check(got, q, k, v, do, mask, causal,
          f"mask {B},{Hq}/{Hkv},N{N},MH{MH},p{density} D{D} causal={causal}")


def test_structured_masks_and_empty_rows():
    """Masks that say what another feature says (lower triangle without the
    causal flag; block diagonal = packed sequences; key columns = key
    lengths), shapes (N, N) and (B, N, N), and whole rows and columns masked
    (empty query rows give o = 0 and zero dQ; masked keys get zero dK, dV)."""
    B, Hq, Hkv, N, D = 2, 4, 2, 300, 128
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, seed=5)
    i, j = np.arange(N)[:, None], np.arange(N)[None, :]
    tril = j <= i
    check(run(q, k, v, do, tril, False), q, k, v, do, tril[None, None], False, "tril (N,N)")
    seg = np.concatenate([np.zeros(100, int), np.ones(77, int), np.full(123, 2)])
    block = np.stack([seg[:, None] == seg[None, :], np.ones((N, N), bool)])  # (B, N, N)
    for causal in (True, False):
        check(run(q, k, v, do, block, causal), q, k, v, do, block[:, None], causal,
              f"block (B,N,N) causal={causal}")
    holes = np.ones((B, 1, N, N), bool)
    holes[0, 0, 17] = False           # an empty query row
    holes[1, 0, :, 250:] = False      # keys past 250 hidden from every row
    holes[1, 0, 40:60, :] = False     # a band of empty rows
    got = run(q, k, v, do, holes, True)
    assert check(got, q, k, v, do, holes, True, "holes") == Hq * 21
    o, _, dq, dk, dv = got
    assert torch.all(dq[0, :, 17] == 0) and torch.all(dq[1, :, 40:60] == 0)
    assert torch.all(dk[1, :, 250:] == 0) and torch.all(dv[1, :, 250:] == 0)


@pytest.mark.parametrize("causal", [True, False])
def test_mask_with_every_other_option(causal):
    """A mask on top of key lengths, ALiBi and a softmax scale (and a sliding
    window when causal), against the oracle with all of them."""
    B, Hq, Hkv, N, D = 2, 4, 2, 517, 64
    rng = np.random.default_rng(21 + causal)
    mask = random_mask(rng, B, Hq, N, 0.6)
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, seed=23 + causal)
    lens = [517, 301]
    slopes = np.array([2.0 ** (-8.0 * (h + 1) / Hq) for h in range(Hq)])
    kw = dict(kv_len=torch.tensor(lens, dtype=torch.int32, device=DEV),
              alibi_slopes=torch.tensor(slopes, dtype=torch.float32, device=DEV),
              softmax_scale=0.1)
    opts = dict(kv_len=lens, alibi=np.float32(slopes).astype(np.float64),
                scale=np.float32(0.1).item())
    if causal:
        kw["sliding_window"] = 90
        opts["window"] = 90
    got = run(q, k, v, do, mask, causal, **kw)
    check(got, q, k, v, do, mask, causal, f"mask+options causal={causal}", **opts)


def test_mask_bf16_bnhd_and_capi():
    """bf16 against the oracle; (B, N, H, D) views bit-identical to the dense
    op; the C ABI (fa_pack_mask, fa_fwd_ex, fa_bwd_ex with mask / mask_t)
    bit-identical to the op; the backward without mask_t is rejected."""
    import fa_p100
    from test_gpu_bf16 import BF_FWD_MAX_ABS, BF_GRAD_REL_L2, bf16_inputs
    B, Hq, Hkv, N, D = 2, 8, 2, 450, 128
    rng = np.random.default_rng(77)
    mask = random_mask(rng, B, 1, N, 0.4)
    m = torch.tensor(mask, device=DEV)
    q, k, v, do = (t.to(DEV) for t in bf16_inputs(B, Hq, Hkv, N, D, seed=17))
    as_bnhd = lambda t: t.transpose(1, 2).contiguous().transpose(1, 2)
    dense = [t.clone().requires_grad_(True) for t in (q, k, v)]
    views = [as_bnhd(t).detach().requires_grad_(True) for t in (q, k, v)]
    o1 = fa_p100.flash_attn(*dense, True, attn_mask=m)
    o2 = fa_p100.flash_attn(*views, True, attn_mask=m)
    o1.backward(do)
    o2.backward(as_bnhd(do))
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)
    for a, b in zip(dense, views):
        assert torch.equal(a.grad, b.grad)
    f = lambda t: t.detach().float().cpu().double().numpy()
    ref_o, _ = ora.attention_fwd(f(q), f(k), f(v), True, mask=mask)
    assert ora.max_abs(f(o1), ref_o) <= BF_FWD_MAX_ABS
    ref = ora.attention_bwd(f(q), f(k), f(v), f(do), True, mask=mask)
    for t, r in zip(dense, ref):
        assert ora.rel_l2(f(t.grad), r) <= BF_GRAD_REL_L2

    lib = load_capi()
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    W = (N + 31) // 32
    bits = torch.empty(B, 1, N, W, dtype=torch.int32, device=DEV)
    bits_t = torch.empty_like(bits)
    assert lib.fa_pack_mask(p(m.to(torch.uint8)), B, N, p(bits), p(bits_t), s) == 0
    opts = fa_opts(dtype=1, mask=bits, mask_t=bits_t, mask_heads=1)
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
    no_t = fa_opts(dtype=1, mask=bits, mask_heads=1)
    assert lib.fa_bwd_ex(p(q), p(k), p(v), p(do), p(o), p(lse), p(dq), p(dk), p(dv), p(ws),
                         ws_bytes, B, Hq, Hkv, N, D, 1, no_t, s) == 10014


def test_hf_hook_masks_match_eager_and_sdpa():
    """Qwen3 through the hook: a 2-D padding mask with holes (keys hidden
    inside rows) against eager with the same mask, and 4-D masks (a boolean
    prefix-LM mask, which is not causal, and its additive float form)
    against sdpa and eager with the same mask; logits at every query row
    that sees a key, within the eager-vs-sdpa envelope."""
    import fa_p100_hf
    from test_gpu_hf import qwen3
    N = 300
    ids = torch.randint(0, 1000, (3, N), device=DEV, generator=torch.Generator(DEV).manual_seed(4))
    holes = torch.ones(3, N, dtype=torch.long, device=DEV)
    holes[0, 10:20] = 0
    holes[1, ::7] = 0
    holes[2, 150:] = 0
    model = qwen3(2, 512, 8, 2, 64, 1024, 1000).eval()

    def logits(impl, mask):
        model.config._attn_implementation = impl
        with torch.no_grad(), torch.autocast("cuda", torch.float16):
            return model(ids, attention_mask=mask).logits.float()

    eager, sdpa = logits("eager", holes), logits("sdpa", holes)
    fa_p100_hf.enable_fa_p100(model)
    fa = logits("fa_p100", holes)
    # Rows that see a real key (causal): every row from the first real token on.
    seen = holes.cumsum(-1) > 0
    env, gap = (sdpa - eager).abs()[seen], (fa - eager).abs()[seen]
    assert gap.mean() <= 2 * env.mean() + 1e-4, (gap.mean().item(), env.mean().item())

    # Prefix-LM: the first 64 tokens see each other, the rest are causal.
    i = torch.arange(N, device=DEV)[:, None]
    j = torch.arange(N, device=DEV)[None, :]
    prefix = ((j <= i) | (j < 64))[None, None].expand(3, 1, N, N)
    additive = torch.zeros(3, 1, N, N, device=DEV).masked_fill(~prefix, torch.finfo(torch.float32).min)
    sd = logits("sdpa", prefix)
    ea = logits("eager", additive)
    fa_b = logits("fa_p100", prefix)
    fa_f = logits("fa_p100", additive)
    env = (sd - ea).abs().mean()
    for got in (fa_b, fa_f):
        assert (got - ea).abs().mean() <= 2 * env + 1e-4, ((got - ea).abs().mean().item(), env)
    # The mask matters: plain causal attention gives other logits.
    causal = logits("fa_p100", None)
    assert (causal - ea).abs().mean() > 4 * env + 1e-3
