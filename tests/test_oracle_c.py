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
    return c


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
