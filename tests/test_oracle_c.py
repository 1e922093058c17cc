"""The C restatement of the oracle (oracle/attention_ref.c, used by the
torch-free driver) against the numpy oracle (oracle/attention.py, which
tests/test_oracle.py pins), plus the reference's finite-difference check of
the C backward (bwd.cu:136-160) through ctypes and through the driver."""
import ctypes
import importlib.util
import os
import subprocess

import numpy as np
import pytest

from helpers import ROOT
from oracle import attention as ora

DRIVER = os.path.join(ROOT, "tests", "driver", "fa_driver")


@pytest.fixture(scope="module")
def lib():
    spec = importlib.util.spec_from_file_location("fa_oracle_build",
                                                  os.path.join(ROOT, "oracle", "build.py"))
    oracle_build = importlib.util.module_from_spec(spec)  # gcc, a fraction of a second
    spec.loader.exec_module(oracle_build)
    path = oracle_build.lib_path()
    if not os.path.exists(path):
        oracle_build.build()
    c = ctypes.CDLL(path)
    dp, i = ctypes.POINTER(ctypes.c_double), ctypes.c_int
    c.ora_fwd.argtypes = [dp] * 5 + [i] * 6
    c.ora_bwd.argtypes = [dp] * 7 + [i] * 6
    c.ora_loss.argtypes = [dp] * 4 + [i] * 6
    c.ora_loss.restype = ctypes.c_double
    c.ora_fwd_ex.argtypes = [dp] * 5 + [i] * 6 + [ctypes.POINTER(OraOpts)]
    c.ora_bwd_ex.argtypes = [dp] * 7 + [i] * 6 + [ctypes.POINTER(OraOpts)]
    c.ora_dropout_threshold.argtypes = [ctypes.c_float]
    c.ora_dropout_threshold.restype = ctypes.c_uint
    c.ora_dropout_keep.argtypes = [ctypes.c_ulonglong, ctypes.c_uint, i, i,
                                   ctypes.POINTER(ctypes.c_ubyte)]
    return c


class OraOpts(ctypes.Structure):
    """ora_opts of oracle/attention_ref.h."""
    _fields_ = [("scale", ctypes.c_double), ("kv_len", ctypes.POINTER(ctypes.c_int)),
                ("window", ctypes.c_int), ("alibi", ctypes.POINTER(ctypes.c_double)),
                ("seg_start", ctypes.POINTER(ctypes.c_int)),
                ("seg_end", ctypes.POINTER(ctypes.c_int)),
                ("mask", ctypes.POINTER(ctypes.c_ubyte)), ("mask_heads", ctypes.c_int),
                ("keep", ctypes.POINTER(ctypes.c_ubyte)), ("drop_scale", ctypes.c_double),
                ("bias", ctypes.POINTER(ctypes.c_double)),
                ("dbias", ctypes.POINTER(ctypes.c_double)),
                ("o", ctypes.POINTER(ctypes.c_double)), ("lse", ctypes.POINTER(ctypes.c_double))]


def _p(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_double))


def _inputs(B, Hq, Hkv, N, D, seed):
    r = np.random.default_rng(seed)
    q = r.standard_normal((B, Hq, N, D))
    k = r.standard_normal((B, Hkv, N, D))
    v = r.standard_normal((B, Hkv, N, D))
    g = r.standard_normal((B, Hq, N, D))
    return q, k, v, g


@pytest.mark.parametrize("B,Hq,Hkv,N,D", [(1, 2, 2, 37, 64), (2, 4, 2, 21, 128), (1, 3, 1, 1, 64)])
@pytest.mark.parametrize("causal", [0, 1])
def test_c_oracle_matches_numpy_oracle(lib, B, Hq, Hkv, N, D, causal):
    q, k, v, g = _inputs(B, Hq, Hkv, N, D, seed=N + D + causal)
    o = np.empty_like(q)
    lse = np.empty((B, Hq, N))
    lib.ora_fwd(_p(q), _p(k), _p(v), _p(o), _p(lse), B, Hq, Hkv, N, D, causal)
    ref_o, ref_lse = ora.attention_fwd(q, k, v, bool(causal))
    np.testing.assert_allclose(o, ref_o, rtol=0, atol=1e-12)
    np.testing.assert_allclose(lse, ref_lse, rtol=0, atol=1e-12)
    dq, dk, dv = np.empty_like(q), np.empty_like(k), np.empty_like(v)
    lib.ora_bwd(_p(q), _p(k), _p(v), _p(g), _p(dq), _p(dk), _p(dv), B, Hq, Hkv, N, D, causal)
    for got, ref in zip((dq, dk, dv), ora.attention_bwd(q, k, v, g, bool(causal))):
        np.testing.assert_allclose(got, ref, rtol=0, atol=1e-11)
    loss = lib.ora_loss(_p(q), _p(k), _p(v), _p(g), B, Hq, Hkv, N, D, causal)
    assert abs(loss - float((g * ref_o).sum())) <= 1e-9 * max(1.0, abs(loss))


def test_c_oracle_backward_is_the_gradient_of_its_loss(lib):
    """Central differences, h = 1e-4 (bwd.cu:136-160), on every element of
    a small causal GQA case."""
    B, Hq, Hkv, N, D, causal, h = 1, 2, 1, 6, 64, 1, 1e-4
    q, k, v, g = _inputs(B, Hq, Hkv, N, D, seed=9)
    dq, dk, dv = np.empty_like(q), np.empty_like(k), np.empty_like(v)
    lib.ora_bwd(_p(q), _p(k), _p(v), _p(g), _p(dq), _p(dk), _p(dv), B, Hq, Hkv, N, D, causal)
    loss = lambda: lib.ora_loss(_p(q), _p(k), _p(v), _p(g), B, Hq, Hkv, N, D, causal)
    for x, an in ((q, dq), (k, dk), (v, dv)):
        flat, aflat = x.reshape(-1), an.reshape(-1)
        for i in range(0, flat.size, 7):
            x0 = flat[i]
            flat[i] = x0 + h
            lp = loss()
            flat[i] = x0 - h
            lm = loss()
            flat[i] = x0
            assert abs((lp - lm) / (2 * h) - aflat[i]) < 1e-6


@pytest.mark.skipif(not os.path.exists(DRIVER), reason="driver not built (tests/driver/build.py)")
def test_driver_finite_difference_mode():
    """fa_driver fd needs no GPU: the C oracle's backward against its loss."""
    p = subprocess.run([DRIVER, "fd"], capture_output=True, text=True, timeout=120)
    assert p.returncode == 0, p.stdout + p.stderr
    assert p.stdout.count(" ok") == 3


def _ptr(a, ctype):
    return a.ctypes.data_as(ctypes.POINTER(ctype))


def _bounds(ids):
    """seg_start / seg_end (B, N) of packed-sequence ids: each token's run."""
    B, N = ids.shape
    start, end = np.zeros((B, N), np.int32), np.zeros((B, N), np.int32)
    for b in range(B):
        i = 0
        while i < N:
            j = i
            while j < N and ids[b, j] == ids[b, i]:
                j += 1
            start[b, i:j], end[b, i:j] = i, j
            i = j
    return start, end


OPTION_SETS = [
    ("kv_len",), ("window",), ("alibi", "scale"), ("segments",), ("mask1",), ("maskH",),
    ("dropout",), ("bias",), ("kv_len", "window", "alibi", "segments", "maskH", "dropout", "bias"),
    ("scale", "mask1", "dropout", "bias"),
]


@pytest.mark.parametrize("saved", [False, True])
@pytest.mark.parametrize("causal", [0, 1])
@pytest.mark.parametrize("opts", OPTION_SETS, ids=lambda o: "+".join(o))
def test_c_oracle_options_match_numpy_oracle(lib, opts, causal, saved):
    """ora_fwd_ex / ora_bwd_ex (the torch-free driver's reference for the
    C ABI's options) against oracle/attention.py (pinned in test_oracle.py)
    on the same options, dbias included, with the backward's P and Dv from a
    saved o and lse or recomputed."""
    if "window" in opts and not causal:
        opts = tuple(o for o in opts if o != "window")
    B, Hq, Hkv, N, D = 2, 4, 2, 23, 16
    q, k, v, g = _inputs(B, Hq, Hkv, N, D, seed=len(opts) + causal)
    r = np.random.default_rng(7 + len(opts))
    o_c = OraOpts()
    kw = {}
    keep_refs = []  # arrays the struct points into
    if "kv_len" in opts:
        lens = np.array([N - 5, 3], np.int32)
        o_c.kv_len, kw["kv_len"] = _ptr(lens, ctypes.c_int), list(lens)
        keep_refs.append(lens)
    if "window" in opts:
        o_c.window, kw["window"] = 4, 4
    if "alibi" in opts:
        slopes = r.uniform(0.05, 0.5, Hq)
        o_c.alibi, kw["alibi"] = _ptr(slopes, ctypes.c_double), slopes
        keep_refs.append(slopes)
    if "scale" in opts:
        o_c.scale, kw["scale"] = 0.21, 0.21
    if "segments" in opts:
        ids = np.sort(r.integers(0, 3, (B, N)), axis=1)
        s0, s1 = _bounds(ids)
        o_c.seg_start, o_c.seg_end = _ptr(s0, ctypes.c_int), _ptr(s1, ctypes.c_int)
        kw["segments"] = ids
        keep_refs += [s0, s1]
    for name, heads in (("mask1", 1), ("maskH", Hq)):
        if name in opts:
            m = r.random((B, heads, N, N)) < 0.75
            m[0, 0, 2] = False  # a row with no key
            mb = np.ascontiguousarray(m, dtype=np.uint8)
            o_c.mask, o_c.mask_heads, kw["mask"] = _ptr(mb, ctypes.c_ubyte), heads, m
            keep_refs.append(mb)
    if "dropout" in opts:
        keep, zs = ora.dropout_keep(11, 0.25, B * Hq, N)
        kb = np.ascontiguousarray(keep, dtype=np.uint8)
        o_c.keep, o_c.drop_scale, kw["dropout"] = _ptr(kb, ctypes.c_ubyte), zs, (keep, zs)
        keep_refs.append(kb)
    if "bias" in opts:
        bias = r.standard_normal((B, Hq, N, N))
        o_c.bias, kw["bias"] = _ptr(bias, ctypes.c_double), bias
        keep_refs.append(bias)
    o, lse = np.empty_like(q), np.empty((B, Hq, N))
    lib.ora_fwd_ex(_p(q), _p(k), _p(v), _p(o), _p(lse), B, Hq, Hkv, N, D, causal,
                   ctypes.byref(o_c))
    ref_o, ref_lse = ora.attention_fwd(q, k, v, bool(causal), **kw)
    np.testing.assert_allclose(o, ref_o, rtol=0, atol=1e-12)
    fin = np.isfinite(ref_lse)
    assert np.array_equal(np.isfinite(lse), fin)
    np.testing.assert_allclose(lse[fin], ref_lse[fin], rtol=0, atol=1e-12)
    bkw = dict(kw)
    if saved:  # a perturbed saved state, used as given by both
        o_s = o + 1e-3 * r.standard_normal(o.shape)
        lse_s = np.where(fin, lse + 1e-3, lse)
        o_c.o, o_c.lse = _p(o_s), _p(lse_s)
        bkw.update(o=o_s, lse=lse_s)
    dq, dk, dv = np.empty_like(q), np.empty_like(k), np.empty_like(v)
    dbias = np.empty((B, Hq, N, N))
    o_c.dbias = _p(dbias)
    lib.ora_bwd_ex(_p(q), _p(k), _p(v), _p(g), _p(dq), _p(dk), _p(dv), B, Hq, Hkv, N, D,
                   causal, ctypes.byref(o_c))
    ref = ora.attention_bwd(q, k, v, g, bool(causal), dbias=True, **bkw)
    for got, want in zip((dq, dk, dv, dbias), ref):
        np.testing.assert_allclose(got, want, rtol=0, atol=1e-11)


@pytest.mark.parametrize("p", [0.0, 0.1, 0.5, 0.9, 0.99999])
def test_c_dropout_draw_matches_numpy_oracle(lib, p):
    """The C restatement of fa_dropout_bits' draw (what the torch-free driver
    checks the GPU's bits against) equals oracle.attention.dropout_keep bit
    for bit, threshold included."""
    for seed, planes, n in ((0, 1, 1), (12345, 3, 37), ((1 << 64) - 3, 2, 64)):
        t = lib.ora_dropout_threshold(p)
        assert t == ora.dropout_threshold(p)
        keep = np.empty((planes, n, n), np.uint8)
        lib.ora_dropout_keep(seed, t, planes, n, _ptr(keep, ctypes.c_ubyte))
        want, _ = ora.dropout_keep(seed, p, planes, n)
        assert np.array_equal(keep.astype(bool), want), (seed, p, planes, n)
