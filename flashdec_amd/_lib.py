"""ctypes binding of ``libflashdec_hip.so`` (declared in ``include/flashdec_hip.h``).

The library is loaded lazily on first use and never replaced by a fallback:
if it is missing or fails to load, every HIP entry point raises
``RuntimeError`` with the reason.  Structures below mirror the C structs
field for field; ``struct_size`` lets the library reject a layout mismatch.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

LIB_NAME = "libflashdec_hip.so"
LIB_PATH = Path(__file__).resolve().with_name(LIB_NAME)

FD_OK = 0
FD_DTYPE_F16 = 0
FD_DTYPE_BF16 = 1
FD_DTYPE_F32 = 2
FD_INDEX_I32 = 0
FD_INDEX_I64 = 1
ABI_VERSION = 9
SPLIT_COUNTER_STRIDE = 64  # FD_SPLIT_COUNTER_STRIDE: uint32 words per (request, KV head) counter
NOALLOC_SCRATCH_BYTES = 8 * 1024 * 1024  # FD_NOALLOC_SCRATCH_BYTES: one stream's scratch slot of fd_paged_decode_noalloc
NOALLOC_STREAM_SLOTS = 4  # FD_NOALLOC_STREAM_SLOTS: slots per GPU (one per stream)
CASCADE_MAX_CHUNK_ROWS = 32  # FD_CASCADE_MAX_CHUNK_ROWS: the larger chunk_rows of fd_cascade_args

_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_vp = ctypes.c_void_p


class PagedDecodeArgs(ctypes.Structure):
    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("dtype", _i32),
        ("num_seqs", _i64),
        ("num_q_heads", _i64),
        ("num_kv_heads", _i64),
        ("head_dim", _i64),
        ("block_size", _i64),
        ("num_blocks", _i64),
        ("max_blocks_per_seq", _i64),
        ("q", _vp),
        ("q_stride", _i64 * 3),
        ("k_cache", _vp),
        ("k_stride", _i64 * 4),
        ("v_cache", _vp),
        ("v_stride", _i64 * 4),
        ("block_tables", _vp),
        ("block_tables_dtype", _i32),
        ("block_tables_stride", _i64 * 2),
        ("seq_lens", _vp),
        ("seq_lens_dtype", _i32),
        ("seq_lens_stride", _i64),
        ("out", _vp),
        ("out_stride", _i64 * 3),
        ("sm_scale", ctypes.c_float),
        ("num_splits", _i32),
        ("split_acc", _vp),
        ("split_acc_stride", _i64 * 4),
        ("split_max", _vp),
        ("split_sum", _vp),
        ("split_stats_stride", _i64 * 3),
        ("split_counters", _vp),
        ("max_seq_len", _i64),
        ("append_k", _vp),
        ("append_k_stride", _i64 * 3),
        ("append_v", _vp),
        ("append_v_stride", _i64 * 3),
        ("slot_mapping", _vp),
        ("slot_mapping_dtype", _i32),
        ("slot_mapping_stride", _i64),
        ("timing_events", _vp * 4),
        ("balance_target", _i32),
        ("kv_reuse", _i32),
        ("rotary_dim", _i32),
        ("rope_base", ctypes.c_double),
        ("rope_cos_sin_table", _vp),
        ("rope_table_rows", _i64),
    ]


class CascadeArgs(ctypes.Structure):
    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("num_groups", _i32),
        ("max_members", _i32),
        ("prefix_splits", _i32),
        ("group_members", _vp),
        ("group_prefix_len", _vp),
        ("row_prefix_len", _vp),
        ("max_prefix_len", _i64),
        ("chunk_rows", _i32),
    ]


class RopeAppendArgs(ctypes.Structure):
    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("dtype", _i32),
        ("batch", _i64),
        ("num_q_heads", _i64),
        ("num_kv_heads", _i64),
        ("head_dim", _i64),
        ("block_size", _i64),
        ("num_blocks", _i64),
        ("rotary_dim", _i64),
        ("base", ctypes.c_double),
        ("q_out", _vp),
        ("q", _vp),
        ("k", _vp),
        ("v", _vp),
        ("k_cache", _vp),
        ("v_cache", _vp),
        ("block_ids", _vp),
        ("block_offsets", _vp),
        ("positions", _vp),
        ("index_dtype", _i32),
        ("cos_sin_table", _vp),
        ("table_rows", _i64),
    ]


EXPORTED_SYMBOLS = (
    "fd_paged_decode",
    "fd_paged_decode_noalloc",
    "fd_paged_decode_noalloc_prepare",
    "fd_paged_decode_cascade",
    "fd_paged_decode_plan",
    "fd_paged_decode_balance_target",
    "fd_fused_rope_kv_append",
    "fd_kv_append",
    "fd_last_error",
    "fd_abi_version",
    "fd_record_launches",
    "fd_last_launch",
)

_lock = threading.Lock()
_lib = None


def library_path() -> Path:
    override = os.environ.get("FLASHDEC_AMD_LIB")
    return Path(override) if override else LIB_PATH


def load_library():
    """Load and type the C-ABI library once; raise RuntimeError if unusable."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = library_path()
        if not path.exists():
            raise RuntimeError(
                f"{path} is not built: the HIP path has no fallback. "
                "Build it with `python -m flashdec_amd._build` (or __graft_entry__.build())."
            )
        try:
            lib = ctypes.CDLL(str(path))
        except OSError as exc:
            raise RuntimeError(f"failed to load {path}: {exc}") from exc
        lib.fd_paged_decode.argtypes = [ctypes.POINTER(PagedDecodeArgs), _vp]
        lib.fd_paged_decode.restype = ctypes.c_int
        lib.fd_paged_decode_noalloc.argtypes = [ctypes.POINTER(PagedDecodeArgs), _vp]
        lib.fd_paged_decode_noalloc.restype = ctypes.c_int
        lib.fd_paged_decode_noalloc_prepare.argtypes = [_vp]
        lib.fd_paged_decode_noalloc_prepare.restype = ctypes.c_int
        lib.fd_paged_decode_cascade.argtypes = [ctypes.POINTER(PagedDecodeArgs), ctypes.POINTER(CascadeArgs), _vp]
        lib.fd_paged_decode_cascade.restype = ctypes.c_int
        lib.fd_paged_decode_balance_target.argtypes = [_i64, _i64]
        lib.fd_paged_decode_balance_target.restype = ctypes.c_int
        lib.fd_paged_decode_plan.argtypes = [_i64, _i64, _i64, _i64, _i64, _i64]
        lib.fd_paged_decode_plan.restype = ctypes.c_int
        lib.fd_fused_rope_kv_append.argtypes = [ctypes.POINTER(RopeAppendArgs), _vp]
        lib.fd_fused_rope_kv_append.restype = ctypes.c_int
        lib.fd_kv_append.argtypes = [ctypes.POINTER(RopeAppendArgs), _vp]
        lib.fd_kv_append.restype = ctypes.c_int
        lib.fd_last_error.argtypes = []
        lib.fd_last_error.restype = ctypes.c_char_p
        lib.fd_abi_version.argtypes = []
        lib.fd_abi_version.restype = ctypes.c_int
        lib.fd_record_launches.argtypes = [ctypes.c_int]
        lib.fd_record_launches.restype = None
        lib.fd_last_launch.argtypes = []
        lib.fd_last_launch.restype = ctypes.c_char_p
        version = lib.fd_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"{path} has ABI version {version}, expected {ABI_VERSION}")
        _lib = lib
        return lib


def record_launches(on: bool = True) -> None:
    """Turn the library's launch record on or off (process-wide; see ``last_launch``)."""
    load_library().fd_record_launches(1 if on else 0)


def last_launch() -> list:
    """Kernels the last library call on this thread launched (demangled names), while the
    launch record is on; no counterpart in the reference."""
    text = load_library().fd_last_launch().decode("utf-8", "replace")
    return text.split(";") if text else []


def check(rc: int, what: str) -> None:
    if rc != FD_OK:
        msg = load_library().fd_last_error().decode("utf-8", "replace")
        raise RuntimeError(f"{what} failed ({rc}): {msg}")


def dtype_code(dtype) -> int:
    import torch

    if dtype == torch.bfloat16:
        return FD_DTYPE_BF16
    if dtype == torch.float16:
        return FD_DTYPE_F16
    if dtype == torch.float32:
        return FD_DTYPE_F32
    raise ValueError(f"unsupported dtype {dtype}")


def index_code(dtype) -> int:
    import torch

    if dtype == torch.int64:
        return FD_INDEX_I64
    if dtype == torch.int32:
        return FD_INDEX_I32
    raise ValueError(f"unsupported index dtype {dtype}")


def current_stream_handle(device) -> int:
    """Raw hipStream_t of torch's current stream on ``device``.

    torch's raw-stream query returns the handle without building a Stream
    object: 0.2 against 1.8 us per call on the MI355X host, a fifth of an
    eager decode call's host time.  The Stream path stays for a torch without
    that query."""
    import torch

    raw = getattr(torch._C, "_cuda_getCurrentRawStream", None)
    if raw is None:
        return torch.cuda.current_stream(device).cuda_stream
    if not isinstance(device, torch.device):
        device = torch.device(device)
    if device.type != "cuda":
        raise ValueError(f"current_stream_handle needs a GPU device, got {device}")
    return raw(torch.cuda.current_device() if device.index is None else device.index)


def paged_decode(args: PagedDecodeArgs, stream: int) -> None:
    lib = load_library()
    args.struct_size = ctypes.sizeof(PagedDecodeArgs)
    check(lib.fd_paged_decode(ctypes.byref(args), stream), "fd_paged_decode")


def paged_decode_noalloc_prepare(stream: int) -> None:
    """``fd_paged_decode_noalloc_prepare``: resolve the scratch address on the stream's device
    (before capturing ``paged_decode_noalloc`` into a graph)."""
    lib = load_library()
    check(lib.fd_paged_decode_noalloc_prepare(stream), "fd_paged_decode_noalloc_prepare")


def paged_decode_noalloc(args: PagedDecodeArgs, stream: int) -> None:
    """``fd_paged_decode_noalloc``: the split partials live in the library's per-GPU scratch."""
    lib = load_library()
    args.struct_size = ctypes.sizeof(PagedDecodeArgs)
    check(lib.fd_paged_decode_noalloc(ctypes.byref(args), stream), "fd_paged_decode_noalloc")


def paged_decode_cascade(args: PagedDecodeArgs, cascade: CascadeArgs, stream: int) -> None:
    lib = load_library()
    args.struct_size = ctypes.sizeof(PagedDecodeArgs)
    cascade.struct_size = ctypes.sizeof(CascadeArgs)
    check(lib.fd_paged_decode_cascade(ctypes.byref(args), ctypes.byref(cascade), stream), "fd_paged_decode_cascade")


def paged_decode_plan(num_seqs, num_q_heads, num_kv_heads, head_dim, max_seq_len, total_seq_len=0) -> int:
    lib = load_library()
    rc = lib.fd_paged_decode_plan(num_seqs, num_q_heads, num_kv_heads, head_dim, max_seq_len, total_seq_len)
    if rc < 0:
        check(rc, "fd_paged_decode_plan")
    return rc


def paged_decode_balance_target(num_seqs, num_kv_heads) -> int:
    lib = load_library()
    rc = lib.fd_paged_decode_balance_target(num_seqs, num_kv_heads)
    if rc < 0:
        check(rc, "fd_paged_decode_balance_target")
    return rc


def rope_append(args: RopeAppendArgs, stream: int, *, rotate: bool) -> None:
    lib = load_library()
    args.struct_size = ctypes.sizeof(RopeAppendArgs)
    if rotate:
        check(lib.fd_fused_rope_kv_append(ctypes.byref(args), stream), "fd_fused_rope_kv_append")
    else:
        check(lib.fd_kv_append(ctypes.byref(args), stream), "fd_kv_append")
