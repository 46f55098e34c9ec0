"""Build the gfx950 shared library.

``build_library()`` compiles every source under ``csrc/`` with hipcc for gfx950 into
``crucible_amd/libcrucible_attn.so`` (objects under ``crucible_amd/_build/``). It also links
``libcrucible_attn_stamps.so``, a diagnostic twin in which the decode and prefill sources are
compiled with ``-DCRUCIBLE_STAMPS`` (per-workgroup phase timestamps, read by
``bench.py --phases``); the product path never loads it.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB_PATH = os.path.join(HERE, "libcrucible_attn.so")
STAMPS_LIB_PATH = os.path.join(HERE, "libcrucible_attn_stamps.so")
STAMPS_SOURCES = ("attn_decode.hip", "attn_prefill.hip")

ARCH = "gfx950"
DEVICE_SOURCES = ["kv_append.hip", "attn_decode.hip", "attn_prefill.hip", "argmax.hip",
                  "model_ops.hip", "abi_common.cpp", "paging.cpp"]
# Packed-FP32 instructions stay off: hipcc would otherwise form v_pk_* f32 ops on its own.
HIPCC_FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
               "-Wall", "-Wno-unused-function"]
# Per-source additions. The decode kernel's leading scalar arguments (the prologue's table,
# length and position pointers, batch and length indexing, the unit plan: 7 arguments, 11
# SGPRs) are preloaded into SGPRs at wave launch, so its first loads do not wait for the
# argument block.
EXTRA_FLAGS = {"attn_decode.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=7"]}


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the crucible_amd library needs ROCm's hipcc")


def _run(cmd):
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n"
                           f"{proc.stdout}\n{proc.stderr}")
    return proc


def _compile_cmd(hipcc, src, obj, defines=()):
    lang = ["-x", "hip"] if src.endswith(".cpp") else []
    return [hipcc, *HIPCC_FLAGS, *EXTRA_FLAGS.get(src, []), *defines, *lang, "-c",
            os.path.join(CSRC, src), "-o", obj]


def _link(hipcc, objs, path):
    tmp = path + ".tmp"
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, path)


def build_library(jobs: int = 8) -> str:
    os.makedirs(BUILD, exist_ok=True)
    hipcc = _hipcc()
    objs = []
    cmds = []
    for src in DEVICE_SOURCES:
        obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
        objs.append(obj)
        cmds.append(_compile_cmd(hipcc, src, obj))
    stamped = {}
    for src in STAMPS_SOURCES:
        stem = os.path.splitext(src)[0]
        stamped[stem + ".o"] = os.path.join(BUILD, stem + "_stamps.o")
        cmds.append(_compile_cmd(hipcc, src, stamped[stem + ".o"], ["-DCRUCIBLE_STAMPS"]))
    with concurrent.futures.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        list(ex.map(_run, cmds))
    _link(hipcc, objs, LIB_PATH)
    _link(hipcc, [stamped.get(os.path.basename(o), o) for o in objs], STAMPS_LIB_PATH)
    return LIB_PATH


def build_all() -> None:
    build_library()


if __name__ == "__main__":
    build_all()
    print(LIB_PATH)
