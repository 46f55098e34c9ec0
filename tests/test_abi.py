"""The C-ABI library loads, exports every symbol include/crucible_attn.h declares, and
rejects invalid arguments before launching anything (no GPU needed for these calls)."""
import ctypes
import os
import re

import pytest

from crucible_amd import _lib


def _declared():
    text = open(_lib.HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(crucible_[a-z0-9_]+)\s*\(", text)))


def test_header_declarations_are_all_bound_and_exported():
    names = _declared()
    assert len(names) >= 28
    lib = _lib.load()
    for name in names:
        assert hasattr(lib, name), f"library does not export {name}"
    assert set(names) == set(_lib.SIGNATURES), "ctypes signatures out of sync with the header"


def test_version():
    assert _lib.load().crucible_attn_version().decode().startswith("crucible_attn")


def test_header_compiles_as_c(tmp_path):
    import subprocess
    src = tmp_path / "t.c"
    src.write_text('#include "crucible_attn.h"\nint main(void){return CRUCIBLE_OK;}\n')
    inc = _lib.HEADER.rsplit("/", 1)[0]
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-I", inc, str(src), "-o",
                    str(tmp_path / "t")], check=True)


def _status_and_msg(rc):
    status, msg = _lib.last_error()
    return rc, status, msg


def test_invalid_arguments_are_rejected_before_launch():
    lib = _lib.load()
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: validation fails first
    # head_dim 64 runs the MFMA kernels, other multiples of 8 up to 256 the generic ones;
    # 100 (not a multiple of 8) and 264 (past 256) are outside this build
    for hd in (100, 264):
        rc = lib.crucible_attention_decode_paged(fake, 1, fake, fake, fake, 0, fake, fake, 1, 12,
                                                 3, hd, 64, 12, 0, 3 * hd, 1024, fake, 1 << 20,
                                                 None)
        assert rc == _lib.ERR_UNSUPPORTED
        assert "head_dim" in _lib.last_error()[1]
        rc = lib.crucible_attention_prefill_paged(fake, 1, fake, fake, fake, 0, fake, 10, 12, 3,
                                                  hd, 12, 0, 3 * hd, 1024, fake, None)
        assert rc == _lib.ERR_UNSUPPORTED
    # layer outside n_layer
    rc = lib.crucible_attention_decode_paged(fake, 1, fake, fake, fake, 0, fake, fake, 1, 12, 3,
                                             64, 64, 12, 12, 192, 1024, fake, 1 << 20, None)
    assert rc == _lib.ERR_INVALID and "layer" in _lib.last_error()[1]
    # n_head not a multiple of n_kv_head
    rc = lib.crucible_attention_prefill_paged(fake, 1, fake, fake, fake, 0, fake, 10, 12, 5, 64,
                                              12, 0, 320, 1024, fake, None)
    assert rc == _lib.ERR_INVALID
    # workspace too small for split-K
    rc = lib.crucible_attention_decode_paged(fake, 1, fake, fake, fake, 0, fake, fake, 16, 12, 3,
                                             64, 128, 12, 0, 192, 2048, fake, 16, None)
    assert rc == _lib.ERR_WORKSPACE
    # bad dtype / pool kind for the append
    rc = lib.crucible_cache_store_rows_paged(fake, 7, fake, 0, fake, fake, 1, 192, 8, 12, 0, None)
    assert rc == _lib.ERR_INVALID
    rc = lib.crucible_cache_store_rows_paged(fake, 0, fake, 9, fake, fake, 1, 192, 8, 12, 0, None)
    assert rc == _lib.ERR_INVALID
    # hybrid prefill needs the chunk's current K/V rows
    rc = lib.crucible_attention_prefill_tiled(fake, 1, fake, fake, None, None, fake, 0, fake, fake,
                                              1, 16, 4, 12, 3, 64, 12, 0, 192, 1, 256, None)
    assert rc == _lib.ERR_INVALID
    # empty batches are a no-op, not an error
    assert lib.crucible_attention_decode_paged(None, 1, None, None, None, 0, None, None, 0, 12, 3,
                                               64, 64, 12, 0, 192, 1024, None, 0, None) == 0


def test_workspace_size_formula():
    lib = _lib.load()
    # a fixed 65536-counter region (256 KiB), the unit plan (2048 entries of 192 int32,
    # 1.5 MiB), then the worst case of 4-page splits: ceil(ceil(2048/16)/4) = 32 splits,
    # 66 floats per (b, h, split)
    assert lib.crucible_attention_decode_workspace_bytes(16, 12, 2048) == (
        65536 * 4 + 2048 * 192 * 4 + 16 * 12 * 32 * 66 * 4)
    assert lib.crucible_attention_decode_workspace_bytes(0, 12, 2048) == 0


def test_decode_step_glue_validates_before_launch():
    lib = _lib.load()
    fake = ctypes.c_void_p(0x1000)  # 16-byte aligned, never dereferenced
    odd = ctypes.c_void_p(0x1004)   # misaligned
    # k_in must be a multiple of 32
    rc = lib.crucible_linear_f64acc(fake, 100, None, 1e-6, fake, 64, 100, None, fake, 64, 4, None)
    assert rc == _lib.ERR_UNSUPPORTED and "k_in" in _lib.last_error()[1]
    # leading dimension below k_in
    rc = lib.crucible_linear_f64acc(fake, 64, None, 1e-6, fake, 64, 128, None, fake, 64, 4, None)
    assert rc == _lib.ERR_INVALID
    # misaligned activations
    rc = lib.crucible_linear_f64acc(odd, 128, None, 1e-6, fake, 64, 128, None, fake, 64, 4, None)
    assert rc == _lib.ERR_INVALID and "aligned" in _lib.last_error()[1]
    # SwiGLU needs its up rows
    rc = lib.crucible_linear_swiglu_f64acc(fake, 128, None, 1e-6, fake, None, 64, 128, fake, 64,
                                           4, None)
    assert rc == _lib.ERR_INVALID
    # zero rows: nothing to do
    assert lib.crucible_linear_f64acc(fake, 128, None, 1e-6, fake, 64, 128, None, fake, 64, 0,
                                      None) == 0
    # RoPE split: an odd head_dim has no pairs, ld too small
    rc = lib.crucible_rope_split_qkv(fake, 1152, fake, fake, fake, fake, fake, fake, 16, 12, 3,
                                     63, 1024, None)
    assert rc == _lib.ERR_UNSUPPORTED
    rc = lib.crucible_rope_split_qkv(fake, 1000, fake, fake, fake, fake, fake, fake, 16, 12, 3,
                                     64, 1024, None)
    assert rc == _lib.ERR_INVALID


def test_greedy_advance_validates_before_launch():
    lib = _lib.load()
    fake = ctypes.c_void_p(0x1000)  # never dereferenced
    args = lambda rows, cols, n_embd, ldx, hist, max_steps, done: (
        fake, rows, cols, fake, n_embd, fake, ldx, fake, hist, fake, max_steps, fake, fake, done,
        None)
    # x rows narrower than the embedding
    assert lib.crucible_greedy_advance(*args(16, 50257, 768, 700, fake, 8, fake)) == _lib.ERR_INVALID
    # negative rows, empty vocabulary
    assert lib.crucible_greedy_advance(*args(-1, 50257, 768, 768, fake, 8, fake)) == _lib.ERR_INVALID
    assert lib.crucible_greedy_advance(*args(16, 0, 768, 768, fake, 8, fake)) == _lib.ERR_INVALID
    # a history of max_steps > 0 rows must exist; the step counter's partner too
    assert lib.crucible_greedy_advance(*args(16, 50257, 768, 768, None, 8, fake)) == _lib.ERR_INVALID
    assert lib.crucible_greedy_advance(*args(16, 50257, 768, 768, fake, 8, None)) == _lib.ERR_INVALID
    # zero rows: nothing to do
    assert lib.crucible_greedy_advance(*args(0, 50257, 768, 768, fake, 8, fake)) == 0


def test_qkv_decode_entry_validates_before_launch():
    lib = _lib.load()
    fake = ctypes.c_void_p(0x1000)
    args = dict(out_dtype=0, batch=16, n_head=12, n_kv=3, hd=64, stride=128, n_layer=12,
                layer=0, kv_dim=192, max_seq=2048)

    def call(row_stride=1152, cos=fake, sin=fake, max_pos=2048, ws_bytes=1 << 22):
        return lib.crucible_attention_decode_qkv_paged_append(
            fake, row_stride, cos, sin, max_pos, fake, fake, fake, args["out_dtype"], fake, fake,
            fake, args["batch"], args["n_head"], args["n_kv"], args["hd"], args["stride"],
            args["n_layer"], args["layer"], args["kv_dim"], args["max_seq"], fake, ws_bytes, None)

    assert call(row_stride=1150) == _lib.ERR_INVALID      # not a multiple of 4
    assert call(row_stride=1100) == _lib.ERR_INVALID      # cannot hold q, k and v
    assert call(cos=None) == _lib.ERR_INVALID             # cos without sin
    assert call(max_pos=1024) == _lib.ERR_INVALID         # tables shorter than max_seq
    assert call(ws_bytes=16) == _lib.ERR_WORKSPACE        # split-K workspace too small


def test_noalloc_limit_is_checked_before_launch():
    """The allocation-free decode's documented limit for batch 16 x 12 query heads is
    max_seq 20,992; one page more (83 splits of 16 pages) returns CRUCIBLE_ERR_WORKSPACE
    before anything touches a device (the pointers here are never dereferenced)."""
    lib = _lib.load()
    fake = ctypes.c_void_p(0x1000)
    for n_kv in (3, 12):
        rc = lib.crucible_attention_decode_paged_append_noalloc(
            fake, _lib.F16, fake, fake, _lib.F32, fake, fake, fake, _lib.F32, fake, fake, fake,
            16, 12, n_kv, 64, 1313, 1, 0, n_kv * 64, 20992 + 16, None)
        assert rc == _lib.ERR_WORKSPACE, n_kv
        assert "static scratch" in _lib.last_error()[1]
        partials = 16 * 12 * 82 * 66 * 4   # the largest call that fits: 82 splits
        assert partials <= (4 << 20) - 32 * 1024 < 16 * 12 * 83 * 66 * 4


def test_tuning_overrides_are_validated_and_restorable():
    """Launch-shape overrides: every key has its environment name, accepts only its
    documented values, and reads back what was set (no GPU involved)."""
    from crucible_amd.gpu import set_tuning, tuning, tuning_state

    lib = _lib.load()
    names = [lib.crucible_attn_tuning_name(k).decode() for k in _lib.TUNE_KEYS.values()]
    assert all(n.startswith("CRUCIBLE_") for n in names) and len(set(names)) == len(names)
    assert lib.crucible_attn_tuning_name(len(_lib.TUNE_KEYS)) is None
    key = _lib.TUNE_KEYS["decode_waves"]
    before = lib.crucible_attn_get_tuning(key)
    assert lib.crucible_attn_set_tuning(key, 5) == _lib.ERR_INVALID
    assert "does not take 5" in _lib.last_error()[1]
    assert lib.crucible_attn_get_tuning(key) == before
    with tuning(decode_waves=4, decode_order="split"):
        assert lib.crucible_attn_get_tuning(key) == 4
        state = tuning_state()
        assert state["CRUCIBLE_DECODE_WAVES"] == 4 and state["CRUCIBLE_DECODE_ORDER"] == 0
    assert lib.crucible_attn_get_tuning(key) == before
    with pytest.raises(_lib.CrucibleError):
        set_tuning(prefill_bufs=5)
    with pytest.raises(_lib.CrucibleError):
        set_tuning(no_such_key=1)


def test_native_caller_compiles_and_links(tmp_path):
    """tests/native_step.cpp, the native caller of the ABI, builds against the header, the
    library and the oracle (host compile only; tests/test_gpu_native_caller.py runs it)."""
    import subprocess

    import native_build

    out = str(tmp_path / "native_step")
    native_build.build(out)
    assert os.path.exists(out)
    nm = subprocess.run(["nm", "-D", "--undefined-only", out], capture_output=True, text=True)
    for sym in ("crucible_attention_decode_paged_append", "crucible_attention_prefill_tiled",
                "crucible_cache_store_packed_paged", "orc_attention_paged_rows"):
        assert sym in nm.stdout, sym
