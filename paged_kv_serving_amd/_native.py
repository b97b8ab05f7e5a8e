"""Build and load the gfx950 C-ABI library ``libpkv.so`` (declared in ``include/pkv.h``).

The library is compiled in-tree with ``hipcc --offload-arch=gfx950`` and loaded with ``ctypes``.
There is no fallback: if the library is missing or fails to load, every operation of the data
path raises :class:`NativeLibraryError`. Nothing here imports torch, so the loader can be
exercised on a machine without a GPU (symbols resolve; no kernel is launched).
"""

from __future__ import annotations

import ctypes
import importlib
import os
import shutil
import subprocess
import sysconfig
import tempfile
import threading
from pathlib import Path

__all__ = [
    "HIPCC_FLAGS",
    "LIB_PATH",
    "SOURCES",
    "EXPORTED_SYMBOLS",
    "NativeLibraryError",
    "PKV_BF16",
    "PKV_F32",
    "build",
    "check",
    "library",
]

PACKAGE_DIR = Path(__file__).resolve().parent
REPO_ROOT = PACKAGE_DIR.parent
CSRC = PACKAGE_DIR / "csrc"
INCLUDE = REPO_ROOT / "include"
LIB_PATH = PACKAGE_DIR / "libpkv.so"
SOURCES = (
    CSRC / "pkv_copy.hip", CSRC / "pkv_rope.hip", CSRC / "pkv_attention.hip", CSRC / "pkv_sample.hip",
    CSRC / "pkv_plan.hip", CSRC / "pkv_model.hip",
)

# gfx950 only. Packed-FP32 VALU instructions are disabled: the code relies on scalar fp32 FMA.
# MFMA accumulators are kept in VGPRs rather than AGPRs: the tile pass rescales its output rows
# with VALU multiplies, which on AGPRs costs a copy out and back per key tile (measured: the
# config-3 tile pass 0.84 -> 0.78 ms).
HIPCC_FLAGS = (
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-mllvm",
    "-amdgpu-mfma-vgpr-form",
)

# pkv_dtype values and pkv_paged_attention flags (include/pkv.h).
PKV_F32 = 0
PKV_BF16 = 1
PKV_ATTN_SHARED_KV = 1
PKV_ATTN_SHORT_ROWS = 2
PKV_ATTN_DOMINANT_TILES = 4
PKV_TILE_WHOLE = -1

PKV_OK = 0
PKV_EINVAL = -1
PKV_ETOOBIG = -4
#: Bytes of the library's static per-device scratch (pkv_paged_attention_noalloc).
STATIC_SCRATCH_BYTES = 64 << 20

EXPORTED_SYMBOLS = (
    "pkv_init",
    "pkv_version",
    "pkv_error_string",
    "pkv_append",
    "pkv_copy_blocks",
    "pkv_rope_append",
    "pkv_attention_workspace_bytes",
    "pkv_tile_head_dim_supported",
    "pkv_paged_attention",
    "pkv_paged_attention_append",
    "pkv_paged_attention_noalloc",
    "pkv_greedy_tokens",
    "pkv_plan_batch",
    "pkv_rms_norm",
    "pkv_silu_mul",
    "pkv_gather_rows",
)


class NativeLibraryError(RuntimeError):
    """The HIP library is missing, failed to load, or returned an error code."""


def _hipcc() -> str:
    found = shutil.which("hipcc")
    if found:
        return found
    candidate = Path(os.environ.get("ROCM_PATH", "/opt/rocm")) / "bin" / "hipcc"
    if candidate.exists():
        return str(candidate)
    raise NativeLibraryError("hipcc not found: the gfx950 library cannot be built")


def build(*, verbose: bool = False) -> Path:
    """Compile every HIP source into ``libpkv.so`` next to this file. Always recompiles.

    The output is written to a temporary file and renamed into place, so a concurrent loader
    never sees a half-written library.
    """
    command = [_hipcc(), *HIPCC_FLAGS, "-I", str(INCLUDE)]
    with tempfile.NamedTemporaryFile(
        dir=PACKAGE_DIR, prefix=".libpkv.", suffix=".so.tmp", delete=False
    ) as handle:
        tmp = Path(handle.name)
    try:
        command += ["-o", str(tmp), *(str(source) for source in SOURCES)]
        result = subprocess.run(command, capture_output=True, text=True, check=False)
        if verbose or result.returncode != 0:
            noise = "packed-fp32-ops"  # the host pass does not know this device feature
            lines = [line for line in result.stderr.splitlines() if noise not in line]
            if lines:
                print("\n".join(lines))
        if result.returncode != 0:
            raise NativeLibraryError(f"hipcc failed with exit code {result.returncode}")
        os.replace(tmp, LIB_PATH)
    finally:
        if tmp.exists():
            tmp.unlink()
    global _LIB
    with _LOCK:
        _LIB = None  # reload on next use
    return LIB_PATH


#: The host helper extension (csrc/pkv_host.cpp): per-entry batch work in C++, no device code.
HOST_SOURCE = CSRC / "pkv_host.cpp"
HOST_PATH = PACKAGE_DIR / f"_pkvhost{sysconfig.get_config_var('EXT_SUFFIX')}"


def build_host(*, verbose: bool = False) -> Path:
    """Compile the ``_pkvhost`` CPython extension next to this file with the host C++ compiler.
    Always recompiles; written to a temporary file and renamed into place."""
    compiler = shutil.which("g++") or shutil.which("c++")
    if compiler is None:
        raise NativeLibraryError("no host C++ compiler: the _pkvhost extension cannot be built")
    with tempfile.NamedTemporaryFile(dir=PACKAGE_DIR, prefix="._pkvhost.", suffix=".so.tmp", delete=False) as handle:
        tmp = Path(handle.name)
    try:
        command = [compiler, "-O3", "-std=c++17", "-shared", "-fPIC", "-Wall", "-Wno-missing-field-initializers",
                   "-I", sysconfig.get_paths()["include"], "-I", str(INCLUDE), "-o", str(tmp),
                   str(HOST_SOURCE)]  # fmt: skip
        result = subprocess.run(command, capture_output=True, text=True, check=False)
        if verbose or result.returncode != 0:
            if result.stderr.strip():
                print(result.stderr)
        if result.returncode != 0:
            raise NativeLibraryError(f"building _pkvhost failed with exit code {result.returncode}")
        os.replace(tmp, HOST_PATH)
    finally:
        if tmp.exists():
            tmp.unlink()
    return HOST_PATH


def host():
    """The ``_pkvhost`` extension module. Raises :class:`NativeLibraryError` if it is not built."""
    if not HOST_PATH.exists():
        raise NativeLibraryError(f"{HOST_PATH} is missing: build it with __graft_entry__.build()")
    return importlib.import_module("paged_kv_serving_amd._pkvhost")


_BOUND = False


def bound_host():
    """:func:`host` with the library's entry points bound into it (``_pkvhost.bind``), so its
    ``plan``, ``paged_attention``, ``paged_attention_append``, ``copy_blocks``, ``rms_norm``,
    ``silu_mul``, ``rope_append``, ``append``, ``forward`` and ``CopyQueue.flush`` call ``libpkv.so``
    directly, and ``stage``, ``forward``, ``CopyQueue.flush`` and ``event_create`` call the
    ``hipMemcpyAsync`` / ``hipGetDevice`` / ``hipSetDevice`` / ``hipEvent*`` functions of the HIP
    runtime ``libpkv.so`` is linked against (looked up through the library's handle, so they are
    that runtime's). Binding loads the library (it must be built)."""
    global _BOUND
    ext = host()
    if not _BOUND:
        lib = library()
        with _LOCK:
            if not _BOUND:
                address = lambda fn: ctypes.cast(fn, ctypes.c_void_p).value  # noqa: E731
                ext.bind(address(lib.pkv_plan_batch), address(lib.pkv_paged_attention),
                         address(lib.pkv_paged_attention_append), address(lib.pkv_copy_blocks),
                         address(lib.pkv_rms_norm), address(lib.pkv_silu_mul),
                         address(lib.pkv_rope_append), address(lib.hipMemcpyAsync),
                         address(lib.pkv_gather_rows), address(lib.pkv_greedy_tokens),
                         address(lib.hipGetDevice), address(lib.hipSetDevice),
                         address(lib.hipEventCreateWithFlags), address(lib.hipEventRecord),
                         address(lib.hipEventSynchronize), address(lib.hipEventDestroy),
                         address(lib.pkv_append))  # fmt: skip
                _BOUND = True
    return ext


_LOCK = threading.Lock()
_LIB: ctypes.CDLL | None = None

_c_int = ctypes.c_int
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_ptr = ctypes.c_void_p


def _declare(lib: ctypes.CDLL) -> None:
    lib.pkv_init.argtypes = [_c_int]
    lib.pkv_init.restype = _c_int
    lib.pkv_version.argtypes = []
    lib.pkv_version.restype = ctypes.c_char_p
    lib.pkv_error_string.argtypes = [_c_int]
    lib.pkv_error_string.restype = ctypes.c_char_p
    lib.pkv_append.argtypes = [
        _ptr, _ptr, _c_int, _i64,  # key_pool, value_pool, pool_dtype, num_slots
        _ptr, _ptr, _c_int,  # new_keys, new_values, src_dtype
        _i64, _i64,  # key_token_stride, value_token_stride
        _ptr, _i64, _i32, _i32,  # slot_mapping, num_tokens, num_heads, head_dim
        _c_int, _ptr,  # device, stream
    ]
    lib.pkv_append.restype = _c_int
    lib.pkv_copy_blocks.argtypes = [
        _ptr, _ptr, _c_int, _ptr, _i64,  # key_pool, value_pool, dtype, pairs, num_pairs
        _i32, _i64, _i64,  # num_layers, num_blocks, block_elems
        _c_int, _ptr,  # device, stream
    ]
    lib.pkv_copy_blocks.restype = _c_int
    lib.pkv_rope_append.argtypes = [
        _ptr, _i64,  # rotated_queries, rotated_token_stride
        _ptr, _ptr, _ptr,  # queries, keys, values
        _i64, _i64, _i64,  # query/key/value token strides
        _ptr, _ptr, _ptr, _i64,  # positions, cos_table, sin_table, table_rows
        _ptr, _ptr, _c_int, _i64,  # key_pool, value_pool, pool_dtype, num_slots
        _ptr, _i64, _i32, _i32,  # slot_mapping, num_tokens, num_heads, head_dim
        _c_int, _ptr,  # device, stream
    ]
    lib.pkv_rope_append.restype = _c_int
    lib.pkv_attention_workspace_bytes.argtypes = [_i64, _i32, _i32, _i32, _i32]
    lib.pkv_attention_workspace_bytes.restype = _i64
    lib.pkv_tile_head_dim_supported.argtypes = [_i32]
    lib.pkv_tile_head_dim_supported.restype = _c_int
    lib.pkv_paged_attention.argtypes = [
        _ptr, _ptr, _i64,  # out, queries, query_token_stride
        _ptr, _ptr, _i64, _ptr,  # query_positions, query_seq, num_queries, caller_rows
        _ptr, _i64, _ptr, _i64,  # rows, num_rows, tiles, num_tiles
        _ptr, _i64,  # merge_rows, num_merge_rows
        _ptr, _ptr, _c_int, _i64, _i32,  # key_cache, value_cache, kv_dtype, num_blocks, block_size
        _ptr, _i32, _ptr, _i32,  # block_tables, block_table_stride, context_lens, num_seqs
        _i32, _i32, ctypes.c_float,  # num_heads, head_dim, scale
        _i32, _i32, _i32,  # max_context_len, partition_size, flags
        _ptr, _i64,  # workspace, workspace_bytes
        _c_int, _ptr,  # device, stream
    ]
    lib.pkv_paged_attention.restype = _c_int
    lib.pkv_paged_attention_noalloc.argtypes = [
        _ptr, _ptr, _i64,  # out, queries, query_token_stride
        _ptr, _ptr, _i64, _ptr,  # query_positions, query_seq, num_queries, caller_rows
        _ptr, _i64, _ptr, _i64,  # rows, num_rows, tiles, num_tiles
        _ptr, _i64,  # merge_rows, num_merge_rows
        _ptr, _ptr, _c_int, _i64, _i32,  # key_cache, value_cache, kv_dtype, num_blocks, block_size
        _ptr, _i32, _ptr, _i32,  # block_tables, block_table_stride, context_lens, num_seqs
        _i32, _i32, ctypes.c_float,  # num_heads, head_dim, scale
        _i32, _i32, _i32,  # max_context_len, partition_size, flags
        _c_int, _ptr,  # device, stream
    ]
    lib.pkv_paged_attention_noalloc.restype = _c_int
    lib.pkv_paged_attention_append.argtypes = [
        _ptr, _ptr, _i64,  # out, queries, query_token_stride
        _ptr, _ptr, _i64, _ptr,  # query_positions, query_seq, num_queries, caller_rows
        _ptr, _i64, _ptr, _i64,  # rows, num_rows, tiles, num_tiles
        _ptr, _i64,  # merge_rows, num_merge_rows
        _ptr, _ptr, _c_int, _i64, _i32,  # key_cache, value_cache, kv_dtype, num_blocks, block_size
        _ptr, _i32, _ptr, _i32,  # block_tables, block_table_stride, context_lens, num_seqs
        _i32, _i32, ctypes.c_float,  # num_heads, head_dim, scale
        _i32, _i32, _i32,  # max_context_len, partition_size, flags
        _ptr, _i64,  # workspace, workspace_bytes
        _ptr, _ptr, _c_int, _i64, _i64, _ptr,  # new_keys, new_values, new_dtype, strides, slot_mapping
        _c_int, _ptr,  # device, stream
    ]
    lib.pkv_paged_attention_append.restype = _c_int
    lib.pkv_greedy_tokens.argtypes = [
        _ptr, _ptr, _i64, _i64, _i64,  # token_ids, logits, row_stride, num_rows, vocab_size
        _c_int, _ptr,  # device, stream
    ]
    lib.pkv_greedy_tokens.restype = _c_int
    lib.pkv_plan_batch.argtypes = [
        _ptr, _ptr, _i64,  # query_seq, query_positions, num_queries
        _ptr, _i32, _ptr, _i32,  # block_tables, stride, context_lens, num_seqs
        _i32, _i32, _i32, _i32,  # block_size, num_heads, head_dim, kv_dtype
        _i32, _i32,  # partition_size, min_tile_rows
        _ptr, _i64, _ptr, _i64, _ptr, _i64,  # rows, capacity, tiles, capacity, merge, capacity
        _ptr, _ptr,  # counts_out, launch_out
    ]
    lib.pkv_plan_batch.restype = _c_int
    lib.pkv_rms_norm.argtypes = [
        _ptr, _i64, _ptr, _i64, _ptr, _i64, _ptr,  # out, stride, hidden, stride, delta, stride, weight
        _i64, _i32, ctypes.c_float, _c_int, _ptr,  # rows, dim, eps, device, stream
    ]
    lib.pkv_rms_norm.restype = _c_int
    lib.pkv_silu_mul.argtypes = [
        _ptr, _i64, _ptr, _ptr, _i64, _i64, _i32, _c_int, _ptr,  # out, stride, gate, up, in stride, rows, width, device, stream
    ]
    lib.pkv_silu_mul.restype = _c_int
    lib.pkv_gather_rows.argtypes = [
        _ptr, _i64, _ptr, _i64, _i64, _ptr, _i64, _i32, _c_int, _ptr,  # out, stride, src, stride, src rows, index, rows, width, device, stream
    ]
    lib.pkv_gather_rows.restype = _c_int


def library() -> ctypes.CDLL:
    """The loaded library. Raises :class:`NativeLibraryError` if it has not been built."""
    global _LIB
    with _LOCK:
        if _LIB is None:
            if not LIB_PATH.exists():
                raise NativeLibraryError(
                    f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                    "(hipcc --offload-arch=gfx950)"
                )
            try:
                lib = ctypes.CDLL(str(LIB_PATH))
            except OSError as error:
                raise NativeLibraryError(f"cannot load {LIB_PATH}: {error}") from error
            _declare(lib)
            _LIB = lib
        return _LIB


_READY: set[int] = set()


def init_device(device: int) -> None:
    """``pkv_init(device)`` once per device: the library's second stream and events, which let a
    call's tile pass run beside its row pass. Later calls are a set lookup."""
    if device in _READY:
        return
    lib = library()
    with _LOCK:
        if device not in _READY:
            check(lib.pkv_init(device), f"pkv_init({device})")
            _READY.add(device)


def check(code: int, what: str) -> None:
    """Raise :class:`NativeLibraryError` for a non-zero PKV_* return code."""
    if code != PKV_OK:
        message = library().pkv_error_string(code).decode()
        raise NativeLibraryError(f"{what} failed: {message} (code {code})")


if __name__ == "__main__":
    print(build(verbose=True))
