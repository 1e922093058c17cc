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
    assert b"64 or 128" in lib.fa_error_string(10001)
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
    assert lib.fa_bwd_workspace_bytes(1, 8, 8, 4096, 80) == 0


def test_capi_validation_returns_before_any_launch():
    lib = load_capi()
    s = ctypes.c_void_p(0)
    z = ctypes.c_void_p(0)
    # head dim, sequence length, heads, batch, null pointers
    assert lib.fa_fwd(z, z, z, z, z, 1, 2, 2, 8, 96, 0, 0, s) == 10001
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
    assert lib.fa_fwd_ex(*([one] * 5), 1, 2, 2, 8, 80, 0, fa_opts(bf16), s) == 10001
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
    # BNHD puts every head of a row in one 32-bit buffer range
    assert lib.fa_fwd_ex(*([one] * 5), 1, 1 << 12, 1, 1 << 14, 128, 0, fa_opts(0, 1), s) == 10007
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


def test_public_api_surface_matches_reference():
    import inspect

    import fa_p100
    import fa_p100_hf
    sig = inspect.signature(fa_p100.flash_attn)
    # The reference's parameters, in order, with its defaults; the extensions
    # (key lengths, sliding window, ALiBi slopes) come after them and default
    # to None, so every reference call binds the same way.
    extensions = ["kv_len", "sliding_window", "alibi_slopes", "segment_ids", "softmax_scale"]
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
