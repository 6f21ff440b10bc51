"""Build libvbmoe.so (HIP, gfx950) in-tree with direct hipcc invocations.

Usage: python build_lib.py [--jobs N]
Output: vbmoe/libvbmoe.so next to this file; objects under _build/.
"""
from __future__ import annotations

import argparse
import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
HOST = HERE / "host"
OUT_DIR = HERE / "vbmoe"
BUILD = HERE / "_build"
LIB = OUT_DIR / "libvbmoe.so"
INCLUDE = HERE.parent / "include"

ARCH = os.environ.get("VBM_OFFLOAD_ARCH", "gfx950")
HIP_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-ffp-contract=off", "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results straight into VGPRs (gfx950 has no need for the AGPR round trip the
    # heuristics otherwise pick when the results feed VALU scale-accumulate code)
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wall", "-Wno-unused-function", "-Wno-unused-command-line-argument",
    f"-I{INCLUDE}", f"-I{CSRC}",
]


def hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found")


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp")) + sorted(HOST.glob("*.cpp"))


# Host-side AddressSanitizer + UndefinedBehaviorSanitizer (the device code is built as usual): a
# CPU-only variant of the library for running the CPU test suite over the host parsers and control
# code (GGUF container parsing, traces, admission, residency replays, the engine-level mirror).
SANITIZE_FLAGS = [
    "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
    "-Xarch_host", "-fno-sanitize-recover=undefined", "-Xarch_host", "-fno-omit-frame-pointer",
]
SANITIZE_DIR = BUILD / "sanitize"
SANITIZE_LIB = SANITIZE_DIR / "libvbmoe.so"


def compile_one(src: Path, sanitize: bool = False) -> Path:
    out_dir = SANITIZE_DIR if sanitize else BUILD
    obj = out_dir / (src.parent.name + "_" + src.name + ".o")
    extra = SANITIZE_FLAGS if sanitize else []
    cmd = [hipcc(), *HIP_FLAGS, *extra, f"-I{HOST}", "-x", "hip", "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"compile failed: {src.name}\n{' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    warnings = [line for line in proc.stderr.splitlines() if "warning" in line and "packed-fp32-ops" not in line]
    if warnings:
        sys.stderr.write(f"[{src.name}]\n" + "\n".join(warnings[:20]) + "\n")
    return obj


def build(jobs: int = 8) -> Path:
    BUILD.mkdir(exist_ok=True)
    OUT_DIR.mkdir(exist_ok=True)
    srcs = sources()
    with concurrent.futures.ThreadPoolExecutor(max_workers=max(1, jobs)) as pool:
        objs = list(pool.map(compile_one, srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs), "-lpthread"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed\n{' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB)
    build_host_tests()
    return LIB


TEST_SRC = HERE.parent / "tests" / "cpp" / "test_native_hip_down.cpp"
TEST_BIN = HERE.parent / "tests" / "cpp" / "bin" / "test_native_hip_down"


def build_host_tests() -> Path:
    """The C++ driver of the engine-level mirror's tests, linked against libvbmoe.so with a
    relative rpath so it runs from any copy of the tree."""
    TEST_BIN.parent.mkdir(parents=True, exist_ok=True)
    cmd = ["g++", "-std=c++17", "-O2", f"-I{HOST}", f"-I{INCLUDE}", str(TEST_SRC), "-o", str(TEST_BIN),
           f"-L{OUT_DIR}", "-lvbmoe", "-Wl,-rpath,$ORIGIN/../../../unified-memory-scheduler_amd/vbmoe"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"host test build failed\n{' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    return TEST_BIN


def build_sanitized(jobs: int = 8) -> Path:
    SANITIZE_DIR.mkdir(parents=True, exist_ok=True)
    with concurrent.futures.ThreadPoolExecutor(max_workers=max(1, jobs)) as pool:
        objs = list(pool.map(lambda src: compile_one(src, True), sources()))
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-shared-libsan", "-fsanitize=address,undefined",
           "-o", str(SANITIZE_LIB), *map(str, objs), "-lpthread"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"sanitized link failed\n{' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    return SANITIZE_LIB


def asan_runtime() -> str:
    out = subprocess.run([hipcc(), "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True, text=True)
    path = out.stdout.strip()
    if not path or not Path(path).exists():
        raise RuntimeError("clang's ASan runtime (libclang_rt.asan-x86_64.so) not found")
    return path


def run_sanitized_suite(pytest_args: list[str]) -> int:
    """The CPU test suite (-m "not gpu") in a child process that loads the sanitized library, with the
    ASan runtime preloaded (the Python interpreter itself is not instrumented, so leak checking is
    off); any ASan report or UBSan finding aborts the run."""
    env = dict(os.environ)
    env["VBM_LIBRARY"] = str(SANITIZE_LIB)
    env["LD_PRELOAD"] = asan_runtime()
    env["ASAN_OPTIONS"] = "detect_leaks=0:abort_on_error=1:halt_on_error=1"
    env["UBSAN_OPTIONS"] = "print_stacktrace=1:halt_on_error=1"
    cmd = [sys.executable, "-m", "pytest", str(HERE.parent / "tests"), "-q", "-m", "not gpu", "-p", "no:cacheprovider",
           *pytest_args]
    return subprocess.run(cmd, env=env, cwd=str(HERE.parent)).returncode


if __name__ == "__main__":
    parser = argparse.ArgumentParser()
    parser.add_argument("--jobs", type=int, default=min(8, os.cpu_count() or 1))
    parser.add_argument("--sanitize", action="store_true",
                        help="build the host-ASan/UBSan variant under _build/sanitize and run the CPU tests on it")
    args, rest = parser.parse_known_args()
    if args.sanitize:
        print(build_sanitized(args.jobs))
        sys.exit(run_sanitized_suite(rest))
    print(build(args.jobs))
