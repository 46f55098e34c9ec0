"""The C ABI driven by a native program, as the reference engine drives its kernels over FFI
(engine/src/gpu_model.rs:1393-1605, :3254-3580): tests/native_step.cpp allocates every
buffer with hipMalloc, runs a packed prefill (packed appends + segment-form attention) and
four decode steps (fused append + decode) on every layer of a 3-layer model, and checks each
launch against the CPU oracle under the reference's element gate and the pools bit for bit.
The binary is built beforehand (__graft_entry__.build(), tests/native_build.py); this test
only runs it, as a child process with a time limit."""
import os
import subprocess

import pytest

from native_build import OUT

pytestmark = pytest.mark.gpu


def test_native_caller_runs_a_prefill_and_decode_steps():
    if not os.path.exists(OUT):
        pytest.fail(f"{OUT} is missing: build it with __graft_entry__.build()")
    print("native caller: running", OUT, flush=True)
    proc = subprocess.run([OUT], capture_output=True, text=True, timeout=120)
    print(proc.stdout[-4000:], flush=True)
    assert proc.returncode == 0, proc.stdout[-2000:] + proc.stderr[-2000:]
    assert "native caller: 0 failed checks" in proc.stdout
    assert proc.stdout.count("bit-identical to the oracle's appends") == 4
    assert proc.stdout.count("0 of ") == 3 + 4 * 3  # prefill layers + decode step layers
