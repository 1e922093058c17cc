"""The torch-free driver (tests/driver/fa_driver) on the GPU: the C ABI with
caller-owned hipMalloc buffers and no torch in the process, checked against
the float64 C oracle over the reference's 4 input regimes and the GQA,
ragged and split-tile shapes, and fa_fwd_ex / fa_bwd_ex with every option
(key lengths, window, ALiBi, scale, packed sequences, a mask packed by
fa_pack_mask, dropout bits from fa_dropout_bits checked against the C draw,
a bias and its gradient) against the C oracle's ora_fwd_ex / ora_bwd_ex; a
benchmark line; the MFMA throughput, MFMA + VALU issue and LDS read probes."""
import os
import re
import subprocess

import pytest

from helpers import ROOT

pytestmark = pytest.mark.gpu

DRIVER = os.path.join(ROOT, "tests", "driver", "fa_driver")


def _run(*args, timeout=100):
    assert os.path.exists(DRIVER), "driver not built: python tests/driver/build.py"
    print("fa_driver", *args, flush=True)
    p = subprocess.run([DRIVER, *args], capture_output=True, text=True, timeout=timeout)
    print(p.stdout[-4000:], p.stderr[-2000:], flush=True)
    return p


def test_driver_check_against_c_oracle():
    p = _run("check")
    assert p.returncode == 0, p.stdout + p.stderr
    assert "check: all ok" in p.stdout
    assert p.stdout.count("| ok") == 28  # 21 plain cases, 7 of the general pair's options


def test_driver_bench_quick():
    p = _run("bench", "quick")
    assert p.returncode == 0, p.stdout + p.stderr
    line = [l for l in p.stdout.splitlines() if l.startswith("C3 headline")][0]
    step_tf = float(line.split()[-1])
    assert step_tf > 100.0, line


def test_driver_mfma_peak_probe():
    p = _run("peak")
    assert p.returncode == 0, p.stdout + p.stderr
    tf = float(re.search(r"sustained ([0-9.]+) TFLOP/s", p.stdout).group(1))
    assert 500.0 < tf <= 2600.0, tf


def test_driver_issue_mix_probe():
    p = _run("mix")
    assert p.returncode == 0, p.stdout + p.stderr
    lines = [l for l in p.stdout.splitlines() if l.startswith("mix:")]
    assert len(lines) == 8, p.stdout
    tf = float(re.search(r"chain alone\s+([0-9.]+) TFLOP/s", p.stdout).group(1))
    assert 500.0 < tf <= 2600.0, tf
    for l in lines:
        cyc = float(re.search(r"([0-9.]+) cycles per", l).group(1))
        assert 0.5 < cyc < 400.0, l


def test_driver_lds_read_probe():
    p = _run("lds")
    assert p.returncode == 0, p.stdout + p.stderr
    rates = [float(x) for x in re.findall(r"([0-9.]+) B/clk per CU", p.stdout)]
    assert len(rates) == 4, p.stdout
    assert all(8.0 < r <= 512.0 for r in rates), rates
