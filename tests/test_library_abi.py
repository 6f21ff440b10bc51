"""CPU-only checks of the product library: it loads, exports every symbol include/vbmoe.h declares,
its host-side generators are deterministic and range-consistent, and the bank layout functions the
device kernels use are a bijection onto each slot (compiled and run on the host)."""
import ctypes as C
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

REPO = Path(__file__).resolve().parents[1]


def test_library_exports_every_declared_symbol(vb):
    lib = vb.load()
    declared = vb.declared_symbols()
    assert len(declared) >= 40
    missing = [name for name in declared if not hasattr(lib, name)]
    assert not missing, missing
    # Every declared function also has a ctypes signature in the binding.
    unbound = [n for n in declared if n not in vb.SIGNATURES and n not in vb.OTHER]
    assert not unbound, unbound
    assert lib.vbm_abi_version() == 1


def test_errors_are_reported_without_a_device(vb):
    lib = vb.load()
    h = C.c_void_p()
    status = lib.vbm_bank_create(12, 32, 64, 1, 0, C.byref(h))     # type 12 is not MXFP4/Q8_0
    assert status == 1 and b"type" in lib.vbm_last_error()
    status = lib.vbm_bank_create(39, 33, 64, 1, 0, C.byref(h))     # rows not a multiple of 32
    assert status == 1 and b"rows" in lib.vbm_last_error()
    status = lib.vbm_bank_create(39, 32, 96, 1, 0, C.byref(h))     # k % 64 != 0
    assert status == 1 and h.value is None


def test_synthetic_generators_are_deterministic_and_range_consistent(vb):
    full = vb.synth_mxfp4(42, 3, 0, 1000)
    part = vb.synth_mxfp4(42, 3, 400, 100)
    assert np.array_equal(full[400 * 17:500 * 17], part)
    assert not np.array_equal(full, vb.synth_mxfp4(43, 3, 0, 1000))
    e = full.reshape(-1, 17)[:, 0]
    assert e.min() == 119 and e.max() == 124            # 127 + U{-8..-3}
    nib = np.concatenate([full.reshape(-1, 17)[:, 1:] & 15, full.reshape(-1, 17)[:, 1:] >> 4]).reshape(-1)
    counts = np.bincount(nib, minlength=16)
    assert counts.min() > 0.8 * counts.mean()           # uniform codes
    q = vb.synth_q8_0(7, 1, 0, 2000).reshape(-1, 34)
    codes = q[:, 2:].view(np.int8)
    assert codes.min() == -127 and codes.max() == 127
    scales = q[:, :2].copy().view(np.float16).astype(np.float32)
    assert scales.min() >= 1e-3 * 0.999 and scales.max() <= 1e-2 * 1.001
    n = vb.synth_normal(1, 2, 0, 200000, 0.0, 0.02)
    assert abs(n.mean()) < 2e-4 and abs(n.std() - 0.02) < 2e-4
    assert np.array_equal(n[1000:1100], vb.synth_normal(1, 2, 1000, 100, 0.0, 0.02))


def test_bank_layout_bijection_host(tmp_path):
    exe = tmp_path / "test_bank_layout"
    subprocess.run(["g++", "-O2", "-std=c++17", f"-I{REPO / 'unified-memory-scheduler_amd' / 'csrc'}",
                    str(REPO / "tests" / "cpp" / "test_bank_layout.cpp"), "-o", str(exe)], check=True)
    proc = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "bijective" in proc.stdout


@pytest.mark.parametrize("args,needle", [(["--gpus", "2"], "exactly one GPU"), (["--tokens", "4"], "single-token")])
def test_bench_refuses_unsupported_runs(args, needle):
    """bench.py measures one GPU at batch 1: other requests exit with status 2 and a message,
    before touching any device."""
    repo = Path(__file__).resolve().parents[1]
    r = subprocess.run([sys.executable, str(repo / "bench.py"), *args], capture_output=True, text=True, timeout=300,
                       cwd=repo)
    assert r.returncode == 2 and needle in r.stderr, (r.returncode, r.stderr[-400:])
