"""Boundary checks that need no GPU: the C-ABI library and the torch binding.

No kernel is launched here: only symbol lookup, host-side helpers and the
argument checks that reject before any device work.
"""
import ctypes

import pytest
import torch

from helpers import LIB, fa_opts, header_functions, load_capi


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(LIB)
    declared = header_functions()
    assert {"fa_fwd", "fa_bwd", "fa_bwd_workspace_bytes", "fa_bwd_preprocess",
            "fa_bwd_main", "fa_error_string", "fa_version"} <= set(declared)
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in include/fa_mi355x.h but not exported"


def test_host_only_helpers():
    lib = load_capi()
    assert lib.fa_version().decode().startswith("fa_mi355x")
    assert lib.fa_error_string(0) == b"success"
    assert b"multiple of 8 from 8 to 256" in lib.fa_error_string(10001)
    assert b"multiple" in lib.fa_error_string(10003)
    # two (B, Hq, N) float32 vectors, each rounded up to 256 bytes; 0 if invalid.
    # dvec + lse2 (256-aligned), counters per key-tile pair (by Hq), then two
    # fp32 dK/dV slots of 128 x D x 2 per pair and (b, kv head).
    assert lib.fa_bwd_workspace_bytes(1, 8, 8, 4096, 128) == (
        2 * 8 * 4096 * 4 + 8 * 16 * 4 + 8 * 16 * 2 * 128 * 128 * 2 * 4)
    assert lib.fa_bwd_workspace_bytes(2, 32, 8, 3001, 128) == (
        2 * 768256 + 2 * 32 * 12 * 4 + 2 * 8 * 12 * 2 * 128 * 128 * 2 * 4)
    assert lib.fa_bwd_workspace_bytes(1, 3, 3, 7, 64) == 512  # one key tile: no pairs
    assert lib.fa_bwd_workspace_bytes(1, 8, 3, 4096, 128) == 0
    assert lib.fa_bwd_workspace_bytes(1, 8, 8, 4096, 100) == 0
    assert lib.fa_bwd_workspace_bytes(1, 8, 8, 4096, 264) == 0
    # head dims 136 .. 256 run at tile width 256 and take its slots
    assert lib.fa_bwd_workspace_bytes(1, 8, 8, 4096, 256) == (
        2 * 8 * 4096 * 4 + 8 * 16 * 4 + 8 * 16 * 2 * 128 * 256 * 2 * 4)
    assert lib.fa_bwd_workspace_bytes(1, 8, 8, 4096, 136) == lib.fa_bwd_workspace_bytes(1, 8, 8, 4096, 256)
    # narrower head dims take the slots of the tile width they run on (80 -> 96)
    assert lib.fa_bwd_workspace_bytes(1, 8, 8, 4096, 80) == lib.fa_bwd_workspace_bytes(1, 8, 8, 4096, 96)


def test_capi_validation_returns_before_any_launch():
    lib = load_capi()
    s = ctypes.c_void_p(0)
    z = ctypes.c_void_p(0)
    # head dim, sequence length, heads, batch, null pointers
    assert lib.fa_fwd(z, z, z, z, z, 1, 2, 2, 8, 100, 0, 0, s) == 10001
    assert lib.fa_fwd(z, z, z, z, z, 1, 2, 2, 8, 4, 0, 0, s) == 10001
    assert lib.fa_fwd(z, z, z, z, z, 1, 2, 2, 8, 264, 0, 0, s) == 10001
    assert lib.fa_fwd(z, z, z, z, z, 1, 2, 2, 8, 256, 0, 0, s) == 10005
    assert lib.fa_fwd(z, z, z, z, z, 1, 2, 2, 8, 136, 0, 0, s) == 10005
    assert lib.fa_fwd(z, z, z, z, z, 1, 2, 2, 0, 64, 0, 0, s) == 10002
    assert lib.fa_fwd(z, z, z, z, z, 1, 4, 3, 8, 64, 0, 0, s) == 10003
    assert lib.fa_fwd(z, z, z, z, z, 0, 2, 2, 8, 64, 0, 0, s) == 10004
    assert lib.fa_fwd(z, z, z, z, z, 1, 2, 2, 8, 64, 0, 0, s) == 10005
    assert lib.fa_bwd_main(*([z] * 5), 0, *([z] * 3), 1, 2, 2, 8, 64, 1, s) == 10005
    assert lib.fa_bwd_preprocess(z, z, z, z, 0, 1, 2, 8, 128, s) == 10005
    one = ctypes.c_void_p(1)
    assert lib.fa_bwd(*([one] * 10), 0, 1, 2, 2, 8, 64, 0, s) == 10006
    # fa_fwd_ex / fa_bwd_ex: the options (element format, layout, window) are
    # checked first, then the same shape, pointer and workspace checks.
    bf16 = 1
    assert lib.fa_fwd_ex(*([one] * 5), 1, 2, 2, 8, 64, 0, fa_opts(bf16, 2), s) == 10008
    assert lib.fa_fwd_ex(*([one] * 5), 1, 2, 2, 8, 64, 0, fa_opts(2, 0), s) == 10009
    assert lib.fa_fwd_ex(*([one] * 5), 1, 2, 2, 8, 100, 0, fa_opts(bf16), s) == 10001
    assert lib.fa_fwd_ex(z, z, z, z, z, 1, 2, 2, 8, 64, 0, fa_opts(bf16, 1), s) == 10005
    assert lib.fa_fwd_ex(z, z, z, z, z, 1, 2, 2, 8, 64, 0, None, s) == 10005  # NULL: defaults
    assert lib.fa_bwd_ex(*([one] * 10), 0, 1, 2, 2, 8, 64, 0, fa_opts(bf16), s) == 10006
    assert lib.fa_bwd_ex(*([one] * 10), 1 << 30, 1, 2, 2, 8, 64, 0, fa_opts(bf16, -1), s) == 10008
    # a window needs causal masking and must not be negative
    assert lib.fa_fwd_ex(*([one] * 5), 1, 2, 2, 8, 64, 0, fa_opts(window=16), s) == 10010
    assert lib.fa_fwd_ex(*([one] * 5), 1, 2, 2, 8, 64, 1, fa_opts(window=-1), s) == 10010
    assert lib.fa_bwd_ex(*([one] * 10), 0, 1, 2, 2, 8, 64, 0, fa_opts(window=4), s) == 10010
    # packed sequences: both bound arrays or neither (causal or not)
    assert lib.fa_fwd_ex(*([one] * 5), 1, 2, 2, 8, 64, 0, fa_opts(seg_start=1), s) == 10011
    assert lib.fa_fwd_ex(*([one] * 5), 1, 2, 2, 8, 64, 1, fa_opts(seg_start=1), s) == 10011
    assert lib.fa_fwd_ex(z, z, z, z, z, 1, 2, 2, 8, 64, 0, fa_opts(seg_start=1, seg_end=1),
                         s) == 10005  # both arrays, non-causal: accepted, then the NULL check
    assert lib.fa_bwd_ex(*([one] * 10), 0, 1, 2, 2, 8, 64, 1, fa_opts(seg_end=1), s) == 10011
    assert b"packed" in lib.fa_error_string(10011)
    # softmax scale: 0 (1/sqrt(D)) or positive and finite
    for bad in (-1.0, float("inf"), float("nan")):
        assert lib.fa_fwd_ex(*([one] * 5), 1, 2, 2, 8, 64, 0, fa_opts(scale=bad), s) == 10012
    assert lib.fa_fwd_ex(z, z, z, z, z, 1, 2, 2, 8, 64, 0, fa_opts(scale=0.3), s) == 10005
    assert b"scale" in lib.fa_error_string(10012)
    # masks: mask_heads 1 or Hq; the backward needs the transposed words too
    assert lib.fa_fwd_ex(*([one] * 5), 1, 4, 2, 8, 64, 0, fa_opts(mask=1, mask_heads=2),
                         s) == 10014
    assert lib.fa_fwd_ex(*([one] * 5), 1, 4, 2, 8, 64, 0, fa_opts(mask=1, mask_heads=0),
                         s) == 10014
    for heads in (1, 4):  # forward: mask alone is enough
        assert lib.fa_fwd_ex(z, z, z, z, z, 1, 4, 2, 8, 64, 1,
                             fa_opts(mask=1, mask_heads=heads), s) == 10005
    assert lib.fa_bwd_ex(*([one] * 10), 1 << 30, 1, 4, 2, 8, 64, 0,
                         fa_opts(mask=1, mask_heads=4), s) == 10014
    assert lib.fa_bwd_ex(*([one] * 10), 0, 1, 4, 2, 8, 64, 0,
                         fa_opts(mask=1, mask_t=1, mask_heads=4), s) == 10006
    assert b"mask_t" in lib.fa_error_string(10014)
    # dropout: a positive finite scale; the backward needs the transposed bits
    for bad in (0.0, -1.0, float("inf"), float("nan")):
        assert lib.fa_fwd_ex(*([one] * 5), 1, 4, 2, 8, 64, 0, fa_opts(drop=1, drop_scale=bad),
                             s) == 10015
    assert lib.fa_fwd_ex(z, z, z, z, z, 1, 4, 2, 8, 64, 1, fa_opts(drop=1, drop_scale=1.25),
                         s) == 10005
    assert lib.fa_bwd_ex(*([one] * 10), 1 << 30, 1, 4, 2, 8, 64, 0,
                         fa_opts(drop=1, drop_scale=1.25), s) == 10015
    assert b"drop_t" in lib.fa_error_string(10015)
    # bias: strides not negative; dbias only with a bias; N <= 2^22 with a bias
    assert lib.fa_fwd_ex(*([one] * 5), 1, 4, 2, 8, 64, 0,
                         fa_opts(bias=1, bias_stride_b=-1), s) == 10016
    big = (1 << 22) + 8  # N * D within 2^29 at D = 8: only the bias bound applies
    assert lib.fa_fwd_ex(*([one] * 5), 1, 1, 1, big, 8, 0, fa_opts(bias=1), s) == 10016
    assert lib.fa_fwd_ex(z, z, z, z, z, 1, 1, 1, big, 8, 0, fa_opts(), s) == 10005
    assert lib.fa_bwd_ex(*([one] * 10), 1 << 30, 1, 4, 2, 8, 64, 0, fa_opts(dbias=1), s) == 10016
    assert lib.fa_fwd_ex(z, z, z, z, z, 1, 4, 2, 8, 64, 1,
                         fa_opts(bias=1, bias_stride_b=0, bias_stride_h=64), s) == 10005
    assert b"dbias" in lib.fa_error_string(10016)
    # no bias at the head dims of tile width 256 (136 .. 256)
    for D in (136, 256):
        assert lib.fa_fwd_ex(*([one] * 5), 1, 4, 2, 8, D, 0, fa_opts(bias=1), s) == 10016
        assert lib.fa_fwd_ex(z, z, z, z, z, 1, 4, 2, 8, D, 0, fa_opts(), s) == 10005
    assert b"head dim up to 128" in lib.fa_error_string(10016)
    # the dropout generator: p in [0, 1), shape, pointers; the scale of the drawn rate
    for draw in (lib.fa_dropout_bits, lib.fa_dropout_bits_causal):
        for bad in (-0.1, 1.0, 1.5, float("nan")):
            assert draw(7, bad, 1, 8, one, one, s) == 10015
        assert draw(7, 0.1, 1, 0, one, one, s) == 10002
        assert draw(7, 0.1, 0, 8, one, one, s) == 10004
        assert draw(7, 0.1, 1, 8, z, one, s) == 10005
    for bad in (-0.1, 1.0, 1.5, float("nan")):
        assert lib.fa_dropout_scale(bad) == 0.0
    for p, t in ((0.0, 0), (0.1, 6554), (0.5, 32768), (0.999999, 65535)):
        assert abs(lib.fa_dropout_scale(p) - 65536.0 / (65536 - t)) < 1e-6 * 65536 / (65536 - t)
    # the packer: N, planes, pointers
    assert lib.fa_pack_mask(one, 1, 0, one, one, s) == 10002
    assert lib.fa_pack_mask(one, 0, 8, one, one, s) == 10004
    assert lib.fa_pack_mask(z, 1, 8, one, None, s) == 10005
    assert lib.fa_pack_mask(one, 1, 8, z, one, s) == 10005
    # BNHD puts every head of a row in one 32-bit buffer range
    assert lib.fa_fwd_ex(*([one] * 5), 1, 1 << 12, 1, 1 << 14, 128, 0, fa_opts(0, 1), s) == 10007
    # kv_rows (key rows != query rows): negative, or combined with packed
    # sequences, a mask, dropout or a bias, is refused; too many rows too.
    assert lib.fa_fwd_ex(*([one] * 5), 1, 2, 2, 8, 64, 1, fa_opts(kv_rows=-1), s) == 10017
    for bad in (fa_opts(kv_rows=9, seg_start=1, seg_end=1),
                fa_opts(kv_rows=9, mask=1, mask_t=1, mask_heads=1),
                fa_opts(kv_rows=9, drop=1, drop_t=1, drop_scale=1.0),
                fa_opts(kv_rows=9, bias=1)):
        assert lib.fa_fwd_ex(*([one] * 5), 1, 2, 2, 8, 64, 1, bad, s) == 10017
    assert lib.fa_fwd_ex(*([one] * 5), 1, 2, 2, 8, 64, 1, fa_opts(kv_rows=1 << 26), s) == 10007
    assert lib.fa_fwd_ex(z, z, z, z, z, 1, 2, 2, 8, 64, 1, fa_opts(kv_rows=9), s) == 10005
    assert lib.fa_fwd_ex(z, z, z, z, z, 1, 2, 2, 8, 64, 1, fa_opts(kv_rows=8, mask=1,
                                                                    mask_heads=1), s) == 10005
    assert b"kv_rows" in lib.fa_error_string(10017)
    # block-sparse lists: not with a mask, a bias or kv_rows != N; the
    # backward needs block_cols; block_cols alone is refused
    for bad in (fa_opts(block_rows=1, mask=1, mask_heads=1), fa_opts(block_rows=1, bias=1),
                fa_opts(block_rows=1, kv_rows=9), fa_opts(block_cols=1)):
        assert lib.fa_fwd_ex(*([one] * 5), 1, 2, 2, 8, 64, 1, bad, s) == 10018
    assert lib.fa_fwd_ex(z, z, z, z, z, 1, 2, 2, 8, 64, 1, fa_opts(block_rows=1), s) == 10005
    assert lib.fa_bwd_ex(*([one] * 10), 1 << 30, 1, 2, 2, 8, 64, 0, fa_opts(block_rows=1),
                         s) == 10018
    assert lib.fa_bwd_ex(*([z] * 10), 1 << 30, 1, 2, 2, 8, 64, 0,
                         fa_opts(block_rows=1, block_cols=1, drop=1, drop_t=1, drop_scale=1.25),
                         s) == 10005
    assert b"block-sparse" in lib.fa_error_string(10018)
    # the block packer: shape, layout planes, pointers
    assert lib.fa_pack_blocks(one, 1, 1, 1, 2, 2, 0, 0, one, one, s) == 10002
    assert lib.fa_pack_blocks(one, 1, 1, 1, 3, 2, 8, 0, one, one, s) == 10003
    assert lib.fa_pack_blocks(one, 1, 1, 0, 2, 2, 8, 0, one, one, s) == 10004
    assert lib.fa_pack_blocks(one, 2, 1, 3, 2, 2, 8, 0, one, one, s) == 10018
    assert lib.fa_pack_blocks(one, 1, 3, 1, 2, 2, 8, 0, one, one, s) == 10018
    assert lib.fa_pack_blocks(z, 1, 1, 1, 2, 2, 8, 0, one, one, s) == 10005
    assert lib.fa_pack_blocks(one, 1, 1, 1, 2, 2, 8, 0, z, one, s) == 10005
    assert b"layout" in lib.fa_error_string(10008)
    assert b"format" in lib.fa_error_string(10009)
    assert b"window" in lib.fa_error_string(10010)


def test_binding_rejects_host_tensors_with_reference_messages():
    import fa_p100
    x = torch.zeros(1, 2, 8, 64, dtype=torch.half)
    with pytest.raises(RuntimeError, match="q must be a CUDA tensor"):
        fa_p100._ext.forward(x, x, x, False, False)
    with pytest.raises(RuntimeError, match="q must be a CUDA tensor"):
        fa_p100._ext.backward(x, x, x, x, x, torch.zeros(1, 2, 8), True)
    with pytest.raises(RuntimeError, match="q must be a CUDA tensor"):
        fa_p100.flash_attn(x, x, x, True)
    # masks: checked on the host before any launch
    with pytest.raises(RuntimeError, match="mask must be a CUDA tensor"):
        fa_p100._ext.pack_mask(torch.ones(8, 8, dtype=torch.bool), True)
    with pytest.raises(ValueError, match="boolean"):
        fa_p100.flash_attn(x, x, x, True, attn_mask=torch.zeros(8, 8))
    with pytest.raises(ValueError, match="attn_mask must be"):
        fa_p100.flash_attn(x, x, x, True, attn_mask=torch.ones(3, 8, 8, dtype=torch.bool))
    with pytest.raises(ValueError, match="packed attn_mask"):
        fa_p100.flash_attn(x, x, x, True, attn_mask=(torch.zeros(1, 2, 8, 2, dtype=torch.int32),) * 2)
    with pytest.raises(ValueError, match="does not combine"):
        fa_p100.flash_attn(x, x, x, True, block_mask=torch.ones(1, 1, dtype=torch.bool),
                           attn_mask=torch.ones(8, 8, dtype=torch.bool))
    with pytest.raises(ValueError, match="block_mask must be"):
        fa_p100.pack_blocks(torch.ones(2, 2, dtype=torch.bool), 1, 2, 2, 8)


def test_public_api_surface_matches_reference():
    import inspect

    import fa_p100
    import fa_p100_hf
    sig = inspect.signature(fa_p100.flash_attn)
    # The reference's parameters, in order, with its defaults; the extensions
    # (key lengths, sliding window, ALiBi slopes, packing, scale, mask) come
    # after them and default to None, so every reference call binds the same way.
    extensions = ["kv_len", "sliding_window", "alibi_slopes", "segment_ids", "softmax_scale",
                  "attn_mask", "dropout_p", "dropout_seed", "attn_bias", "block_mask"]
    assert list(sig.parameters)[:5] == ["q", "k", "v", "causal", "full_precision"]
    assert sig.parameters["causal"].default is False
    assert sig.parameters["full_precision"].default is False
    assert list(sig.parameters)[5:] == extensions
    assert all(sig.parameters[n].default is None for n in extensions)
    for name in ("_FlashAttnP100", "reference", "_expand_kv", "_ext"):
        assert hasattr(fa_p100, name)
    for name in ("fa_p100_attention_forward", "register", "enable_fa_p100", "_set_impl"):
        assert hasattr(fa_p100_hf, name)
    assert callable(fa_p100._ext.forward) and callable(fa_p100._ext.backward)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("B,Hq,Hkv,N,D", [(2, 4, 4, 37, 64), (1, 8, 2, 64, 128),
                                           (2, 4, 1, 19, 64)])
def test_reference_helper_matches_the_oracle(B, Hq, Hkv, N, D, causal, dtype):
    """fa_p100.reference (fa_p100.py:58-75's plain-torch attention, re-shipped
    for users' own checks) against the float64 oracle, itself pinned against
    torch SDPA, finite differences and closed forms in test_oracle.py: MHA,
    GQA and MQA, causal and dense, fp32 and fp16 inputs. The result is
    rounded to the input dtype, so the bar is that dtype's rounding of
    |O| <= max|V| plus the fp32 arithmetic; a wrong head map (tile instead of
    repeat_interleave) or a flipped causal mask is caught too."""
    import numpy as np

    import fa_p100
    from oracle import attention as ora
    g = torch.Generator().manual_seed(B * 1000 + Hq * 100 + N)
    q, k, v = (torch.randn(B, h, N, D, generator=g).to(dtype) for h in (Hq, Hkv, Hkv))
    got = fa_p100.reference(q, k, v, causal)
    assert got.dtype == dtype and got.shape == q.shape
    f64 = lambda t: t.double().numpy()
    ref, _ = ora.attention_fwd(f64(q), f64(k), f64(v), causal)
    tol = 2e-3 if dtype == torch.float16 else 2e-5
    assert ora.max_abs(f64(got), ref) <= tol
    # Planted mistakes the bar must see: the wrong GQA head map, and the
    # mask flipped to the other triangle.
    if Hq != Hkv and Hkv > 1:
        tiled = lambda t: t.repeat(1, Hq // Hkv, 1, 1)
        wrong, _ = ora.attention_fwd(f64(q), f64(tiled(k)), f64(tiled(v)), causal)
        assert ora.max_abs(f64(got), wrong) > 10 * tol
    if causal:
        flip = lambda t: t.flip(2)
        wrong, _ = ora.attention_fwd(f64(flip(q)), f64(flip(k)), f64(flip(v)), True)
        assert ora.max_abs(f64(got), np.flip(wrong, 2)) > 10 * tol


def test_shape_limits_follow_the_one_dimensional_grids():
    """Every launch is a 1-D grid, so B*Hq is not bounded by a 65535 grid.y
    any more: B*Hq = 65536 (and well beyond) passes validation. What is
    bounded is each launch's work-item count (workgroups x threads), which
    the dispatch packet holds in 32 bits, and N*D (a head's rows within 2^30
    bytes);
    fa_bwd_workspace_bytes returns 0 exactly for a shape validation rejects."""
    lib = load_capi()
    for B, Hq, Hkv, N, D in [(1, 65536, 65536, 64, 64), (2, 32768, 8, 128, 128),
                             (65536, 1, 1, 1, 64), (1, 1, 1, 1 << 20, 128),
                             (1, 1, 1, 1 << 22, 128)]:
        assert lib.fa_bwd_workspace_bytes(B, Hq, Hkv, N, D) > 0, (B, Hq, Hkv, N, D)
    # 2^23 query heads of 4096 rows need more than 2^32 forward work-items.
    assert lib.fa_bwd_workspace_bytes(1 << 13, 1 << 10, 1 << 10, 4096, 128) == 0
    # At a tile width (32, 64, 96, 128) a head's rows, with the 256 rows a
    # staged tile may address past them, stay within 2^32 bytes: (N+256)*D
    # <= INT_MAX; narrower head dims keep (N+256)*D <= 2^29.
    for D in (32, 64, 96, 128, 256):
        n_max = (2**31 - 1) // D - 256
        assert lib.fa_bwd_workspace_bytes(1, 1, 1, n_max, D) > 0, D
        assert lib.fa_bwd_workspace_bytes(1, 1, 1, n_max + 1, D) == 0, D
    for D in (8, 40, 120, 136, 248):
        n_max = 2**29 // D - 256
        assert lib.fa_bwd_workspace_bytes(1, 1, 1, n_max, D) > 0, D
        assert lib.fa_bwd_workspace_bytes(1, 1, 1, n_max + 1, D) == 0, D


def test_bnhd_limit_spans_every_head_of_a_row():
    """The (B, N, H, D) layout reads a head through one buffer range over all
    H heads of each row. At a tile width the limit is (N+256)*H*D <= INT_MAX:
    32 heads of 128 at N = 262144 (N*H*D = 2^30, above the 2^29 bound that
    narrow head dims keep) pass validation and stop at the null pointers."""
    lib = load_capi()
    s = ctypes.c_void_p(0)
    z = ctypes.c_void_p(0)
    assert lib.fa_fwd_bnhd(z, z, z, z, z, 1, 32, 8, 1 << 18, 128, 1, s) == 10005
    assert lib.fa_fwd_bnhd(z, z, z, z, z, 1, 64, 8, 1 << 18, 128, 1, s) == 10007
    assert lib.fa_fwd_bnhd(z, z, z, z, z, 1, 32, 8, 1 << 18, 120, 1, s) == 10007
    n_max = (2**31 - 1) // (32 * 128) - 256
    assert lib.fa_fwd_bnhd(z, z, z, z, z, 1, 32, 8, n_max, 128, 1, s) == 10005
    assert lib.fa_fwd_bnhd(z, z, z, z, z, 1, 32, 8, n_max + 1, 128, 1, s) == 10007
