"""C ABI checks that need no GPU: the library loads, exports exactly what
``include/flashdec_hip.h`` declares, and the ctypes mirrors of the argument
structs have the layout a C compiler gives the header."""

import ctypes
import re
import shutil
import subprocess
from pathlib import Path

import pytest

from flashdec_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "flashdec_hip.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:int|void|const\s+char\s*\*)\s*(fd_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_exactly_the_bound_symbols():
    assert declared_functions() == sorted(_lib.EXPORTED_SYMBOLS)


def test_library_loads_and_exports_every_declared_symbol():
    if not _lib.LIB_PATH.exists():
        pytest.fail(f"{_lib.LIB_PATH} is not built; run __graft_entry__.build()")
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    for name in declared_functions():
        assert hasattr(lib, name), name
    lib.fd_abi_version.restype = ctypes.c_int
    assert lib.fd_abi_version() == _lib.ABI_VERSION
    lib.fd_last_error.restype = ctypes.c_char_p
    assert isinstance(lib.fd_last_error(), bytes)


def test_timeline_stamps_exist_in_the_measurement_build_only():
    """The per-wave timeline stamps (``-DFD_TIMELINE``) are compiled into
    ``libflashdec_timeline.so`` for bench.py's timeline workloads; the product
    library exports no stamp buffer, and the measurement build exports the same
    C ABI beside it."""
    from flashdec_amd import _build

    if not _lib.LIB_PATH.exists() or not _build.TIMELINE_LIB_PATH.exists():
        pytest.fail("the libraries are not built; run __graft_entry__.build()")
    product = ctypes.CDLL(str(_lib.LIB_PATH))
    timeline = ctypes.CDLL(str(_build.TIMELINE_LIB_PATH))
    assert not hasattr(product, "fd_timeline_buffer")
    assert hasattr(timeline, "fd_timeline_buffer")
    for name in declared_functions():
        assert hasattr(timeline, name), name


def test_library_rejects_bad_arguments_without_touching_a_device():
    lib = _lib.load_library()
    args = _lib.PagedDecodeArgs()
    args.struct_size = ctypes.sizeof(args) - 8  # wrong ABI size is refused before any HIP call
    rc = lib.fd_paged_decode(ctypes.byref(args), None)
    assert rc == -1
    assert b"struct_size" in lib.fd_last_error()
    assert lib.fd_paged_decode(None, None) == -1
    rope = _lib.RopeAppendArgs()
    rope.struct_size = 3
    assert lib.fd_fused_rope_kv_append(ctypes.byref(rope), None) == -1
    assert lib.fd_kv_append(ctypes.byref(rope), None) == -1
    # the cascade entry point validates both structs before any HIP call
    args.struct_size = ctypes.sizeof(args) - 8
    cas = _lib.CascadeArgs()
    cas.struct_size = ctypes.sizeof(cas)
    assert lib.fd_paged_decode_cascade(ctypes.byref(args), ctypes.byref(cas), None) == -1
    assert b"fd_paged_decode_cascade" in lib.fd_last_error() and b"struct_size" in lib.fd_last_error()
    assert lib.fd_paged_decode_cascade(None, ctypes.byref(cas), None) == -1


LAYOUT_PROBE = r"""
#include <stddef.h>
#include <stdio.h>
#include "flashdec_hip.h"
#define F(S, f) printf(#S " " #f " %zu\n", offsetof(S, f));
int main(void) {
  printf("fd_paged_decode_args sizeof %zu\n", sizeof(fd_paged_decode_args));
  printf("fd_rope_append_args sizeof %zu\n", sizeof(fd_rope_append_args));
  printf("fd_cascade_args sizeof %zu\n", sizeof(fd_cascade_args));
%s
  return 0;
}
"""


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not available")
def test_ctypes_structs_match_c_layout(tmp_path):
    pairs = [("fd_paged_decode_args", _lib.PagedDecodeArgs), ("fd_rope_append_args", _lib.RopeAppendArgs),
             ("fd_cascade_args", _lib.CascadeArgs)]
    lines = [f"  F({c}, {name})" for c, py in pairs for name, _ in py._fields_]
    src = tmp_path / "probe.c"
    src.write_text(LAYOUT_PROBE.replace("%s", "\n".join(lines)))
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", "-I", str(HEADER.parent), str(src), "-o", str(exe)],
                   check=True)
    c_layout = {}
    for line in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.splitlines():
        struct, field, value = line.split()
        c_layout[(struct, field)] = int(value)
    for c, py in pairs:
        assert c_layout[(c, "sizeof")] == ctypes.sizeof(py), c
        for name, _ in py._fields_:
            assert c_layout[(c, name)] == getattr(py, name).offset, (c, name)


def test_header_constants_match_binding():
    text = HEADER.read_text()
    consts = dict(re.findall(r"#define\s+(FD_\w+)\s+\(?(-?\d+)\)?", text))
    assert int(consts["FD_ABI_VERSION"]) == _lib.ABI_VERSION
    assert int(consts["FD_SPLIT_COUNTER_STRIDE"]) == _lib.SPLIT_COUNTER_STRIDE
    assert int(consts["FD_DTYPE_F16"]) == _lib.FD_DTYPE_F16
    assert int(consts["FD_DTYPE_BF16"]) == _lib.FD_DTYPE_BF16
    assert int(consts["FD_DTYPE_F32"]) == _lib.FD_DTYPE_F32
    assert int(consts["FD_INDEX_I64"]) == _lib.FD_INDEX_I64
    assert int(consts["FD_NOALLOC_SCRATCH_BYTES"]) == _lib.NOALLOC_SCRATCH_BYTES
    assert int(consts["FD_NOALLOC_STREAM_SLOTS"]) == _lib.NOALLOC_STREAM_SLOTS
    assert int(consts["FD_CASCADE_MAX_CHUNK_ROWS"]) == _lib.CASCADE_MAX_CHUNK_ROWS


def _noalloc_args(num_seqs, num_q_heads, head_dim, num_splits):
    args = _lib.PagedDecodeArgs()
    args.struct_size = ctypes.sizeof(args)
    args.dtype = _lib.FD_DTYPE_BF16
    args.num_seqs, args.num_q_heads, args.num_kv_heads = num_seqs, num_q_heads, 2
    args.head_dim, args.block_size, args.num_blocks, args.max_blocks_per_seq = head_dim, 32, 1, 1
    args.num_splits = num_splits
    return args


def test_noalloc_rejects_a_workspace_and_oversized_launches_before_any_hip_call():
    lib = _lib.load_library()
    args = _noalloc_args(8, 16, 128, 16)
    args.split_acc = 0x1000  # never dereferenced: the call is refused first
    assert lib.fd_paged_decode_noalloc(ctypes.byref(args), None) == -1
    assert b"must be NULL" in lib.fd_last_error()
    args = _noalloc_args(8, 16, 128, 16)
    args.split_counters = 0x1000
    assert lib.fd_paged_decode_noalloc(ctypes.byref(args), None) == -1
    assert b"must be NULL" in lib.fd_last_error()
    # B64 Hq16 D128 S16: 64*16*16*130*4 bytes of partials > 8 MiB
    args = _noalloc_args(64, 16, 128, 16)
    assert lib.fd_paged_decode_noalloc(ctypes.byref(args), None) == -1
    msg = lib.fd_last_error()
    assert b"exceed" in msg and str(_lib.NOALLOC_SCRATCH_BYTES).encode() in msg
    # one split more than fits at B8 Hq16 D128 (126 fit)
    args = _noalloc_args(8, 16, 128, 127)
    assert lib.fd_paged_decode_noalloc(ctypes.byref(args), None) == -1
    assert b"exceed" in lib.fd_last_error()
    args.struct_size -= 8
    assert lib.fd_paged_decode_noalloc(ctypes.byref(args), None) == -1
    assert b"struct_size" in lib.fd_last_error()
    assert lib.fd_paged_decode_noalloc(None, None) == -1
