"""Guards on the machine code of the built library (CPU only, no GPU): properties of the
decode kernels that the HIP source states only through the compiler's behaviour, so that a
compiler update that moves them fails here rather than only in the GPU tests.

The split combine publishes each split's partial with write-through (sc1) stores, waits
until they are acknowledged (s_waitcnt vmcnt(0)), passes the workgroup barrier and only
then increments the unit's counter with a returning agent-scope atomic; the combining
split reads the partials with sc1 loads. These are plain stores and a relaxed atomic, not
a release/acquire pair, so the wait between them is what orders them. The kernel's first
seven arguments are preloaded into SGPRs (-amdgpu-kernarg-preload-count=7, 12 SGPRs).

The gfx950 code object is taken from the library's .hip_fatbin section with ROCm's
llvm-objcopy, clang-offload-bundler and llvm-objdump: this build's own code.
"""
import os
import re
import subprocess

import pytest

from crucible_amd import _build

ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
LLVM = os.path.join(ROCM, "llvm", "bin")
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"
TARGET = f"hipv4-amdgcn-amd-amdhsa--{_build.ARCH}"


def _tool(name):
    path = os.path.join(LLVM, name)
    if not os.path.exists(path):
        pytest.skip(f"{name} not found under {LLVM}")
    return path


def _run(*cmd):
    proc = subprocess.run(cmd, capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr[-2000:]
    return proc.stdout


@pytest.fixture(scope="module")
def decode_code_object(tmp_path_factory):
    """Path of the gfx950 code object holding the decode kernels, and their symbol names."""
    if not os.path.exists(_build.LIB_PATH):
        pytest.skip("the library is not built")
    tmp = tmp_path_factory.mktemp("codeobj")
    fatbin = tmp / "fatbin.bin"
    _run(_tool("llvm-objcopy"), f"--dump-section=.hip_fatbin={fatbin}", _build.LIB_PATH,
         str(tmp / "lib_copy.so"))
    data = fatbin.read_bytes()
    starts = [m.start() for m in re.finditer(re.escape(MAGIC), data)]
    assert starts, "no offload bundle in .hip_fatbin"
    bundler, objdump = _tool("clang-offload-bundler"), _tool("llvm-objdump")
    for k, start in enumerate(starts):
        end = starts[k + 1] if k + 1 < len(starts) else len(data)
        bundle = tmp / f"bundle{k}.bin"
        bundle.write_bytes(data[start:end])
        co = tmp / f"bundle{k}.co"
        _run(bundler, "--unbundle", "--type=o", f"--targets={TARGET}", f"--input={bundle}",
             f"--output={co}")
        names = [line.split()[-1] for line in _run(objdump, "-t", str(co)).splitlines()
                 if "decode_kernel" in line]
        kernels = sorted(n for n in names if n.endswith("DecodeArgsE") and "decode_kernelI" in n)
        if kernels:
            return co, kernels
    pytest.fail("no decode_kernel in the library's gfx950 code objects")


def _disassemble(co, symbols):
    """{symbol: [instruction text, ...]} for the given functions (or kernel descriptors)."""
    out = _run(_tool("llvm-objdump"), "-D", f"--mcpu={_build.ARCH}",
               "--disassemble-symbols=" + ",".join(symbols), str(co))
    funcs, cur = {}, None
    for line in out.splitlines():
        m = re.match(r"^[0-9a-f]+ <(.+)>:$", line)
        if m:
            cur = funcs.setdefault(m.group(1), [])
        elif cur is not None and line.strip():
            cur.append(line.split("//")[0].strip())
    return funcs


def _publish_order_problem(name, ins):
    """None if the in-kernel combine of `ins` (a function's instructions in address order)
    waits for its published partials before the counter, else what is wrong; "" when the
    function has no combine (no returning atomic add)."""
    atomics = [i for i, t in enumerate(ins)
               if re.match(r"(global|buffer|flat)_atomic_add\b", t) and " sc0" in t]
    if not atomics:
        return ""
    a = atomics[0]
    barriers = [i for i in range(a) if ins[i].startswith("s_barrier")]
    if not barriers:
        return f"{name}: no barrier before the counter atomic"
    b = barriers[-1]
    stores = [i for i in range(b) if re.match(r"(global|buffer)_store", ins[i])
              and " sc1" in ins[i]]
    if not stores:
        return f"{name}: no write-through partial store before the counter"
    s = stores[-1]
    waits = [t for t in ins[s + 1:b] if t.startswith("s_waitcnt")
             and ("vmcnt(0)" in t or re.fullmatch(r"s_waitcnt\s+0", t))]
    if not waits:
        return (f"{name}: no vmcnt(0) between the last published store and the barrier "
                f"before the counter:\n" + "\n".join(ins[s:a + 1]))
    if not any(re.match(r"(global|buffer)_load", t) and " sc1" in t for t in ins[a + 1:]):
        return f"{name}: the combine does not read the partials with sc1 loads"
    return None


def test_decode_kernels_wait_for_the_published_partials_before_counting(decode_code_object):
    co, kernels = decode_code_object
    funcs = _disassemble(co, kernels)
    checked = 0
    for name in kernels:
        problem = _publish_order_problem(name, funcs[name])
        assert not problem, problem
        checked += problem is None
    assert checked > 0, "no decode kernel with the in-kernel combine found"
    print(f"{checked} of {len(kernels)} decode kernels combine in-kernel; all wait")


# the publish sequence as the built kernels have it (abridged)
_GOOD = ["buffer_store_dwordx4 v[2:5], v11, s[36:39], 0 offen sc1",
         "global_store_dword v[6:7], v10, off sc1",
         "s_waitcnt vmcnt(0) expcnt(0) lgkmcnt(0)",
         "s_barrier",
         "global_atomic_add v2, v1, v2, s[6:7] sc0",
         "s_waitcnt vmcnt(0)",
         "s_barrier",
         "buffer_load_dwordx4 v[18:21], v1, s[36:39], 0 offen sc1"]


def test_the_order_check_rejects_a_missing_or_partial_wait():
    """The check passes the built order and fails it with the wait taken out or weakened."""
    assert _publish_order_problem("good", _GOOD) is None
    no_wait = [t for t in _GOOD if not t.startswith("s_waitcnt vmcnt(0) expcnt")]
    assert "no vmcnt(0)" in _publish_order_problem("no wait", no_wait)
    partial = [("s_waitcnt vmcnt(1)" if t.startswith("s_waitcnt vmcnt(0) expcnt") else t)
               for t in _GOOD]
    assert "no vmcnt(0)" in _publish_order_problem("partial wait", partial)
    plain_loads = [t.replace(" sc1", "") if t.startswith("buffer_load") else t for t in _GOOD]
    assert "sc1 loads" in _publish_order_problem("plain loads", plain_loads)
    assert _publish_order_problem("no combine", _GOOD[:2]) == ""


def test_decode_kernels_preload_their_leading_arguments(decode_code_object):
    co, kernels = decode_code_object
    descs = _disassemble(co, [k + ".kd" for k in kernels])
    for name in kernels:
        text = "\n".join(descs.get(name + ".kd", []))
        m = re.search(r"\.amdhsa_user_sgpr_kernarg_preload_length\s+(\d+)", text)
        assert m, f"{name}: no kernarg preload in its descriptor"
        assert int(m.group(1)) >= 11, f"{name}: preload length {m.group(1)}"
