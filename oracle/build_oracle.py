"""Build recipes for the CPU oracle (test infrastructure only).

  liboracle:  oracle/libvbm_oracle.so from oracle/vbm_oracle.c (gcc, -ffp-contract=off, OpenMP).
  reference:  oracle/_ref/* compiled directly from the reference repository's own sources
              (read in place under REF_ROOT, never copied):
                - libref_mxfp4_vnni.so  <- tools/trace/cpu_mxfp4_vnni.cpp (exports
                  ggml_vec_dot_mxfp4_q8_0; needs an AVX512VL+VNNI host to run)
                - libref_f32_experts.so <- tools/engine/f32_experts.cpp with oracle/ref_f32_experts_shim.cpp
                  (exports ref_glu: the reference executor's own activation stage)
                - test_expert_dispatch  <- tests/test_expert_dispatch.cpp linked against this
                  repository's ExpertPlan (unified-memory-scheduler_amd/host/expert_dispatch.cpp)
                - test_expert_dispatch_asan  <- the same, built with -fsanitize=address,undefined
              The reference build is skipped (with a message) when REF_ROOT is absent.

Usage: python oracle/build_oracle.py [--no-ref]
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
REPO = HERE.parent
REF_ROOT = Path(os.environ.get("VBM_REFERENCE_ROOT", "/root/reference"))
LIB = HERE / "libvbm_oracle.so"
REF_OUT = HERE / "_ref"
HOST_DIR = REPO / "unified-memory-scheduler_amd" / "host"


def run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed: {' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")


def build_oracle() -> Path:
    tmp = LIB.with_suffix(".so.tmp")
    run(["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-fopenmp", "-ffp-contract=off", "-fno-fast-math",
         "-Wall", "-Wextra", "-Wno-unused-parameter", str(HERE / "vbm_oracle.c"), "-o", str(tmp), "-lm"])
    os.replace(tmp, LIB)
    return LIB


def build_reference() -> list[Path]:
    if not REF_ROOT.exists():
        print(f"reference sources not present at {REF_ROOT}; skipping oracle/_ref", file=sys.stderr)
        return []
    REF_OUT.mkdir(exist_ok=True)
    built = []
    vnni = REF_OUT / "libref_mxfp4_vnni.so"
    run(["g++", "-O2", "-std=c++20", "-fPIC", "-shared", "-mavx2", "-mfma", "-mf16c", "-mavx512f", "-mavx512vl",
         "-mavx512vnni", "-mavxvnni", "-ffp-contract=off", str(REF_ROOT / "tools/trace/cpu_mxfp4_vnni.cpp"),
         "-o", str(vnni)])
    built.append(vnni)
    f32 = REF_OUT / "libref_f32_experts.so"
    run(["g++", "-O2", "-std=c++20", "-fPIC", "-shared", "-ffp-contract=off", f"-I{REF_ROOT / 'tools/engine'}",
         str(HERE / "ref_f32_experts_shim.cpp"), str(REF_ROOT / "tools/engine/f32_experts.cpp"), "-o", str(f32)])
    built.append(f32)
    dispatch = REF_OUT / "test_expert_dispatch"
    run(["g++", "-O2", "-std=c++20", "-ffp-contract=off", "-pthread", f"-I{HOST_DIR}",
         str(REF_ROOT / "tests/test_expert_dispatch.cpp"), str(HOST_DIR / "expert_dispatch.cpp"), "-o", str(dispatch)])
    built.append(dispatch)
    # the same test under host AddressSanitizer + UndefinedBehaviorSanitizer (the ExpertPlan indexes
    # by caller data)
    dispatch_asan = REF_OUT / "test_expert_dispatch_asan"
    run(["g++", "-O1", "-g", "-std=c++20", "-ffp-contract=off", "-pthread", "-fsanitize=address,undefined",
         "-fno-sanitize-recover=undefined", "-fno-omit-frame-pointer", f"-I{HOST_DIR}",
         str(REF_ROOT / "tests/test_expert_dispatch.cpp"), str(HOST_DIR / "expert_dispatch.cpp"), "-o", str(dispatch_asan)])
    built.append(dispatch_asan)
    return built


if __name__ == "__main__":
    print(build_oracle())
    if "--no-ref" not in sys.argv:
        for path in build_reference():
            print(path)
