"""The library's pre-launch argument validation under AddressSanitizer and UBSan (CPU only).

tests/abi_validation.cpp calls every C-ABI entry point with fake device pointers, first with
ordinary arguments, then with each integer argument replaced by extreme values, and checks
the statuses the header documents. Here it is linked against the library's own sources
compiled with the sanitizers on the host code (hipcc, each -fsanitize after -Xarch_host;
the device code is compiled as usual and never runs) and against tests/hip_stub.cpp, a HIP
runtime with no device, so no call can reach a GPU; any signed overflow, out-of-bounds
access or leak in the validation code aborts the run. The objects are cached in
tests/_build/sanitized/ and rebuilt when a source is newer; the first build takes about a
minute.
"""
import os
import subprocess
from concurrent.futures import ThreadPoolExecutor

import pytest

from crucible_amd import _build

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
OUT = os.path.join(HERE, "_build", "sanitized")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
SOURCES = ("attn_decode.hip", "attn_prefill.hip", "kv_append.hip", "argmax.hip",
           "model_ops.hip", "abi_common.cpp", "paging.cpp")
HOST_SAN = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
            "-Xarch_host", "-fno-sanitize-recover=all", "-Xarch_host", "-fno-omit-frame-pointer"]


def _newer(src, obj):
    return not os.path.exists(obj) or os.path.getmtime(src) > os.path.getmtime(obj)


def _build_driver() -> str:
    hipcc = os.path.join(ROCM, "bin", "hipcc")
    clang = os.path.join(ROCM, "llvm", "bin", "clang++")
    if not (os.path.exists(hipcc) and os.path.exists(clang)):
        pytest.skip("ROCm's hipcc and clang++ are needed to build the sanitized library")
    os.makedirs(OUT, exist_ok=True)
    headers = [os.path.join(_build.CSRC, f) for f in os.listdir(_build.CSRC)
               if f.endswith((".hpp", ".h"))] + [os.path.join(ROOT, "include", "crucible_attn.h")]
    newest_header = max(os.path.getmtime(h) for h in headers)
    flags = ["-O1", "-g", "-std=c++17", "-fPIC", f"--offload-arch={_build.ARCH}",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-I", _build.CSRC, "-I", os.path.join(ROOT, "include")]
    jobs = []
    objs = []
    for src in SOURCES:
        path = os.path.join(_build.CSRC, src)
        obj = os.path.join(OUT, os.path.splitext(src)[0] + ".o")
        objs.append(obj)
        if _newer(path, obj) or os.path.getmtime(obj) < newest_header:
            jobs.append([hipcc, *flags, *HOST_SAN, "-x", "hip", "-c", path, "-o", obj])

    def run(cmd):
        return subprocess.run(cmd, capture_output=True, text=True)

    with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as pool:
        for proc in pool.map(run, jobs):
            assert proc.returncode == 0, proc.stderr[-3000:]
    exe = os.path.join(OUT, "abi_validation")
    driver = os.path.join(HERE, "abi_validation.cpp")
    stub = os.path.join(HERE, "hip_stub.cpp")
    if any(_newer(o, exe) for o in objs) or _newer(driver, exe) or _newer(stub, exe):
        proc = subprocess.run([clang, "-O1", "-g", "-std=c++17", "-D__HIP_PLATFORM_AMD__",
                               "-I", os.path.join(ROCM, "include"),
                               "-I", os.path.join(ROOT, "include"),
                               "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
                               driver, stub, *objs, "-o", exe],
                              capture_output=True, text=True)
        assert proc.returncode == 0, proc.stderr[-3000:]
    return exe


@pytest.mark.timeout(600)
def test_validation_of_every_entry_point_under_sanitizers():
    exe = _build_driver()
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:halt_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    proc = subprocess.run([exe], capture_output=True, text=True, timeout=300, env=env)
    out = proc.stdout + proc.stderr
    assert proc.returncode == 0, out[-6000:]
    assert "AddressSanitizer" not in out and "runtime error" not in out, out[-6000:]
    assert " 0 failed;" in proc.stdout, proc.stdout[-3000:]
