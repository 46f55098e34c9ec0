"""Build recipe of tests/native_step.cpp, the native (C++) caller of the C ABI.

Host code only: g++ against ROCm's HIP runtime headers, linked with the product library
and the CPU oracle (test infrastructure), both found at run time through $ORIGIN-relative
run paths, so the binary runs from any copy of the repository. __graft_entry__.build()
calls build() (tests/_build/native_step); test_gpu_native_caller.py runs it.
"""
from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
OUT = os.path.join(HERE, "_build", "native_step")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")


def command(out: str = OUT) -> list[str]:
    return [os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-Wall", "-Wextra",
            "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(ROCM, "include"),
            os.path.join(HERE, "native_step.cpp"), "-o", out,
            "-L", os.path.join(ROOT, "crucible_amd"), "-lcrucible_attn",
            "-L", os.path.join(ROOT, "oracle", "_build"), "-loracle",
            "-L", os.path.join(ROCM, "lib"), "-lamdhip64",
            "-Wl,-rpath,$ORIGIN/../../crucible_amd", "-Wl,-rpath,$ORIGIN/../../oracle/_build",
            "-Wl,-rpath," + os.path.join(ROCM, "lib")]


def build(out: str = OUT) -> str:
    os.makedirs(os.path.dirname(out), exist_ok=True)
    subprocess.run(command(out), check=True, capture_output=True, text=True)
    return out
