"""The C-ABI library builds for gfx950, loads, and exports exactly what include/pkv.h declares.

Runs without a GPU: only host-side entry points are called (version, error strings, workspace
sizing) plus argument checks that return before any HIP call.
"""

from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from paged_kv_serving_amd import _native

ROOT = Path(__file__).resolve().parents[1]


def declared_functions() -> list[str]:
    text = (ROOT / "include" / "pkv.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pkv_[a-z_0-9]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not _native.LIB_PATH.exists():
        _native.build()
    return _native.library()


def test_every_declared_function_is_exported(lib) -> None:
    names = declared_functions()
    assert names == sorted(_native.EXPORTED_SYMBOLS)
    out = subprocess.run(["nm", "-D", "--defined-only", str(_native.LIB_PATH)], capture_output=True, text=True, check=True)
    exported = {line.split()[-1] for line in out.stdout.splitlines() if " T " in line}
    for name in names:
        assert name in exported, name
        assert getattr(lib, name) is not None


def test_the_library_holds_gfx950_code_only() -> None:
    blob = _native.LIB_PATH.read_bytes()  # built in-tree from csrc/ by _native.build()
    assert b"amdgcn-amd-amdhsa--gfx950" in blob
    for other in (b"gfx942", b"gfx90a", b"gfx908", b"sm_"):
        assert b"amdgcn-amd-amdhsa--" + other not in blob


def test_version_and_error_strings(lib) -> None:
    assert lib.pkv_version().decode().startswith("pkv ")
    assert lib.pkv_error_string(0) == b"ok"
    assert lib.pkv_error_string(-1) == b"invalid argument"
    assert lib.pkv_error_string(-2) == b"unsupported shape or dtype"
    assert lib.pkv_error_string(-3).startswith(b"HIP")
    assert lib.pkv_error_string(7) == b"unknown error code"


def test_workspace_sizing(lib) -> None:
    # one partition -> no workspace
    assert lib.pkv_attention_workspace_bytes(64, 32, 128, 512, 512) == 0
    # 4096 / 512 = 8 partitions of (128 + 2) floats per (query, head)
    assert lib.pkv_attention_workspace_bytes(64, 32, 128, 4096, 512) == 64 * 32 * 8 * 130 * 4
    assert lib.pkv_attention_workspace_bytes(64, 32, 128, 4097, 0) == 64 * 32 * 9 * 130 * 4
    assert lib.pkv_attention_workspace_bytes(1, 1, 128, 100, 17) == -1  # not a multiple of 16
    assert lib.pkv_attention_workspace_bytes(1, 1, 128, 100, 2048) == -1  # above 1024


def test_bad_arguments_are_refused_before_any_device_work(lib) -> None:
    null = None
    # num_heads = 0
    assert lib.pkv_append(null, null, 0, 10, null, null, 0, 8, 8, null, 1, 0, 8, 0, null) == -1
    # bf16 source into a float32 pool is not a supported conversion
    assert lib.pkv_append(null, null, 0, 10, null, null, 1, 8, 8, null, 1, 1, 8, 0, null) == -2
    # a value stride shorter than a row
    assert lib.pkv_append(null, null, 0, 10, null, null, 0, 8, 4, null, 1, 1, 8, 0, null) == -1
    # zero tokens is a no-op
    assert lib.pkv_append(null, null, 0, 10, null, null, 0, 8, 8, null, 0, 1, 8, 0, null) == 0
    # unknown dtype
    assert lib.pkv_copy_blocks(null, null, 9, null, 1, 1, 4, 16, 0, null) == -1
    assert lib.pkv_copy_blocks(null, null, 0, null, 0, 1, 4, 16, 0, null) == 0
    # partition size not a multiple of 16
    args = [null, null, 8, null, null, 1, null, null, 0, null, 0, null, -1, null, null, 0, 4, 4, null, 1,
            null, 1, 1, 8, ctypes.c_float(0.5), 8, 17, 0, null, 0, 0, null]  # fmt: skip
    assert lib.pkv_paged_attention(*args) == -1
    args[26] = 16
    args[27] = 2
    assert lib.pkv_paged_attention(*args) == -1  # unknown flag
    args[27] = 1
    assert lib.pkv_paged_attention(*args) == -1  # null pointers
    args[27] = 0
    args[12] = -2
    assert lib.pkv_paged_attention(*args) == -1  # a merge count below -1
    args[12] = 3
    assert lib.pkv_paged_attention(*args) == -1  # merge rows counted but not given
    assert lib.pkv_tile_head_dim_supported(128) == 1
    assert lib.pkv_tile_head_dim_supported(16) == 0


def test_gather_rows_arguments_are_refused_before_any_device_work(lib) -> None:
    fake = ctypes.c_void_p(4096)
    assert lib.pkv_gather_rows(fake, 8, fake, 8, 10, fake, 0, 8, 0, None) == 0  # no rows: nothing to do
    assert lib.pkv_gather_rows(fake, 4, fake, 8, 10, fake, 2, 8, 0, None) == -1  # out stride below width
    assert lib.pkv_gather_rows(fake, 8, fake, 4, 10, fake, 2, 8, 0, None) == -1  # src stride below width
    assert lib.pkv_gather_rows(fake, 8, fake, 8, 10, fake, 2, 0, 0, None) == -1  # width 0
    assert lib.pkv_gather_rows(None, 8, fake, 8, 10, fake, 2, 8, 0, None) == -1  # null output


def test_rope_append_arguments_are_refused_before_any_device_work(lib) -> None:
    # Placeholder addresses: every call below returns before touching them or the device.
    fake = [ctypes.c_void_p(4096 * (i + 1)) for i in range(9)]
    rot, q, k, v, pos, cos, sin, kp, vp = fake
    slots = ctypes.c_void_p(4096 * 20)

    def call(rot_stride=64, strides=(64, 64, 64), dtype=0, tokens=2, heads=2, dim=32, q_ptr=q, **kw):
        return lib.pkv_rope_append(
            kw.get("rot", rot), rot_stride, q_ptr, k, v, *strides, pos, cos, sin, 16, kp, vp,
            dtype, 100, slots, tokens, heads, dim, 0, None,
        )  # fmt: skip

    assert call(dim=31) == -1  # odd head_dim
    assert call(heads=0) == -1
    assert call(dtype=7) == -1  # unknown pool dtype
    assert call(tokens=-1) == -1
    assert call(tokens=0) == 0  # nothing to do
    assert call(strides=(63, 64, 64)) == -1  # a token stride shorter than a row
    assert call(rot_stride=32) == -1
    assert call(rot=q, rot_stride=64, strides=(192, 192, 192)) == -1  # in place needs equal strides
    assert call(q_ptr=None) == -1  # null pointer


def test_greedy_tokens_arguments_are_refused_before_any_device_work(lib) -> None:
    out, logits = ctypes.c_void_p(4096), ctypes.c_void_p(8192)
    assert lib.pkv_greedy_tokens(out, logits, 8, 2, 0, 0, None) == -1  # empty vocabulary
    assert lib.pkv_greedy_tokens(out, logits, 7, 2, 8, 0, None) == -1  # stride shorter than a row
    assert lib.pkv_greedy_tokens(out, logits, 8, -1, 8, 0, None) == -1
    assert lib.pkv_greedy_tokens(out, logits, 8, 0, 8, 0, None) == 0  # no rows: nothing to do
    assert lib.pkv_greedy_tokens(None, logits, 8, 2, 8, 0, None) == -1


def test_missing_library_fails_loudly(tmp_path, monkeypatch) -> None:
    monkeypatch.setattr(_native, "LIB_PATH", tmp_path / "absent.so")
    monkeypatch.setattr(_native, "_LIB", None)
    with pytest.raises(_native.NativeLibraryError, match="missing"):
        _native.library()


def test_fused_append_arguments_are_refused_before_any_device_work(lib) -> None:
    # Placeholder addresses: every call below returns before touching them or the device.
    fake = [ctypes.c_void_p(4096 * (i + 1)) for i in range(12)]
    out, q, qpos, qseq, kc, vc, tables, ctx, ws, nk, nv, slots = fake

    def call(new_keys=nk, new_values=nv, new_dtype=0, key_stride=512, value_stride=512,
             pool_dtype=0, slot_mapping=slots, head_dim=128):  # fmt: skip
        return lib.pkv_paged_attention_append(
            out, q, 4 * head_dim, qpos, qseq, 3, None, None, 0, None, 0, None, -1, kc, vc, pool_dtype, 100, 16,
            tables, 8, ctx, 3, 4, head_dim, ctypes.c_float(0.1), 100, 0, 0, ws, 1 << 20,
            new_keys, new_values, new_dtype, key_stride, value_stride, slot_mapping, 0, None,
        )  # fmt: skip

    assert call(new_keys=None) == -1
    assert call(slot_mapping=None) == -1
    assert call(new_dtype=1, pool_dtype=0) == -2  # bfloat16 rows into a float32 pool
    assert call(new_dtype=5) == -1
    assert call(key_stride=100) == -1  # shorter than a token row (4 heads x 128)
    assert call(key_stride=514) == -2  # rows not 16-byte aligned


def test_init_refuses_device_ordinals_out_of_range(lib) -> None:
    einval = -1  # PKV_EINVAL
    assert lib.pkv_init(-1) == einval
    assert lib.pkv_init(64) == einval


@pytest.mark.gpu
def test_init_is_idempotent_on_a_device(device) -> None:
    lib = _native.library()
    assert lib.pkv_init(device.index) == 0
    assert lib.pkv_init(device.index) == 0


def test_model_ops_refuse_bad_arguments_before_any_launch(lib) -> None:
    """pkv_rms_norm / pkv_silu_mul validate sizes, strides and eps on the host (no HIP call)."""
    einval = _native.PKV_EINVAL
    one = ctypes.c_void_p(16)  # never dereferenced: every call below fails its checks first
    assert lib.pkv_rms_norm(one, 4, one, 4, None, 0, one, 1, 0, 1e-5, 0, None) == einval  # dim 0
    assert lib.pkv_rms_norm(one, 3, one, 4, None, 0, one, 1, 4, 1e-5, 0, None) == einval  # out stride
    assert lib.pkv_rms_norm(one, 4, one, 4, one, 2, one, 1, 4, 1e-5, 0, None) == einval  # delta stride
    assert lib.pkv_rms_norm(one, 4, one, 4, None, 0, one, 1, 4, -1.0, 0, None) == einval  # eps < 0
    assert lib.pkv_rms_norm(None, 4, one, 4, None, 0, one, 1, 4, 1e-5, 0, None) == einval  # null out
    assert lib.pkv_rms_norm(None, 4, None, 4, None, 0, None, 0, 4, 1e-5, 0, None) == _native.PKV_OK  # no rows
    assert lib.pkv_silu_mul(one, 4, one, one, 8, 1, 0, 0, None) == einval  # width 0
    assert lib.pkv_silu_mul(one, 4, one, one, 3, 1, 4, 0, None) == einval  # input stride
    assert lib.pkv_silu_mul(None, 4, one, one, 8, 1, 4, 0, None) == einval  # null out
    assert lib.pkv_silu_mul(None, 4, None, None, 8, 0, 4, 0, None) == _native.PKV_OK  # no rows
