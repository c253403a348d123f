"""CPU checks of the C ABI: the library loads, exports every declared symbol, and the
ctypes mirrors of the structs match the C layout.  No compute calls (no GPU here)."""
import ctypes
import os
import re
import subprocess

import pytest
import torch

from phasekv_amd import _lib

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))
HEADER = os.path.join(ROOT, "include", "phasekv_hip.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pk_[a-z_0-9]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    declared = _declared_functions()
    assert len(declared) >= 12
    for name in declared:
        assert hasattr(lib, name), name
    assert set(declared) == set(_lib.exported_symbols())


def test_version_and_error_string_do_not_need_a_gpu():
    lib = _lib.load()
    assert b"gfx950" in lib.pk_version()
    assert isinstance(lib.pk_last_error(), bytes)


def test_struct_layout_matches_c(tmp_path):
    src = tmp_path / "layout.c"
    src.write_text(r'''
#include <stddef.h>
#include <stdio.h>
#include "phasekv_hip.h"
#define F(T, f) printf(#T "." #f " %zu\n", offsetof(T, f));
int main(void) {
  printf("pk_segment %zu\n", sizeof(pk_segment));
  printf("pk_decode_problem %zu\n", sizeof(pk_decode_problem));
  F(pk_segment, seq_lens) F(pk_segment, k_data) F(pk_segment, v_mins)
  F(pk_segment, k_data_bstride) F(pk_segment, tok_stride)
  F(pk_decode_problem, q) F(pk_decode_problem, segments) F(pk_decode_problem, num_segments)
  F(pk_decode_problem, table) F(pk_decode_problem, table_count) F(pk_decode_problem, table_bits)
  return 0;
}
''')
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)],
                   check=True)
    out = dict(line.rsplit(" ", 1) for line in
               subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
               if line)
    assert int(out["pk_segment"]) == ctypes.sizeof(_lib.PkSegment)
    assert int(out["pk_decode_problem"]) == ctypes.sizeof(_lib.PkDecodeProblem)
    for key, val in out.items():
        if "." in key:
            struct, field = key.split(".")
            cls = _lib.PkSegment if struct == "pk_segment" else _lib.PkDecodeProblem
            assert getattr(cls, field).offset == int(val), key


def test_python_side_rejects_bad_arguments_before_any_launch():
    from phasekv_amd.kernels import packing
    x = torch.zeros(1, 2, 8, 8, dtype=torch.float16)
    with pytest.raises(ValueError, match="bits"):
        packing.quantize_pack(x, 3, -1, 4)
    with pytest.raises(ValueError, match="uint8"):
        packing.pack_low_bits(torch.zeros(3, dtype=torch.int32), 2)
    with pytest.raises(ValueError):
        packing._vals_per_byte(5)
    # no CPU path: a host tensor is refused, not computed with torch
    with pytest.raises(ValueError, match="ROCm GPU"):
        packing.quantize_pack(x, 2, -1, 4)


def test_transposed_storage_only_for_the_second_innermost_axis():
    """The ABI refuses transposed code / scale storage for any other axis, before any launch."""
    lib = _lib.load()
    shape = _lib.i64_array((2, 64, 32))
    strides = _lib.i64_array((64 * 32, 32, 1))
    rc = lib.pk_quantize_pack(None, _lib.PK_DTYPE_F16, 3, shape, strides, 2, 2, 32, None, None,
                              None, _lib.PK_LAYOUT_META_TRANSPOSED, None)
    assert rc == _lib.PK_ERR_INVALID
    assert b"axis == ndim - 2" in lib.pk_last_error()
    rc = lib.pk_quantize_pack(None, _lib.PK_DTYPE_F16, 3, shape, strides, 1, 2, 32, None, None,
                              None, 7, None)
    assert rc == _lib.PK_ERR_INVALID



def test_merge_partial_sets_rejects_bad_sets_before_any_launch():
    """pk_merge_partial_sets validates every set on the host: no launch (and so no GPU)
    is reached by a bad call."""
    lib = _lib.load()
    fake = 1 << 32                                     # never dereferenced on these paths

    def call(sets, nsets, outer=5, inner=8, hd=64, out=fake):
        arr = (_lib.PkPartialSet * max(1, len(sets)))(*sets)
        return lib.pk_merge_partial_sets(arr, nsets, outer, inner, hd, out, None, None, None,
                                         None)

    ok = _lib.PkPartialSet(fake, fake, fake, 40, 2, 0, 8, 1)       # last row 4 * 8 + 7 = 39
    cases = [
        ([ok], 0, {}, "partial sets"),
        ([ok] * 5, 5, {}, "partial sets"),
        ([ok], 1, {"hd": 48}, "head_dim"),
        ([ok], 1, {"hd": 2}, "head_dim"),
        ([ok], 1, {"out": None}, "no output"),
        ([_lib.PkPartialSet(fake, fake, fake, 40, 2, 0, 1, 6)], 1, {}, "past its rows"),
        ([_lib.PkPartialSet(fake, fake, fake, 40, 0, 0, 8, 1)], 1, {}, "n > 0"),
        ([_lib.PkPartialSet(fake, 0, fake, 40, 2, 0, 8, 1)], 1, {}, "null partials"),
        ([_lib.PkPartialSet(fake, fake, fake + 4, 40, 2, 0, 8, 1)], 1, {}, "16-byte aligned"),
    ]
    for sets, nsets, kw, msg in cases:
        assert call(sets, nsets, **kw) == _lib.PK_ERR_INVALID, msg
        assert msg.encode() in lib.pk_last_error(), (msg, lib.pk_last_error())
    # and the Python wrapper refuses host tensors (no CPU path) and more than four sets
    from phasekv_amd import decode as dec
    m, l, acc = torch.zeros(4, 2), torch.ones(4, 2), torch.zeros(4, 2, 8)
    with pytest.raises(ValueError, match="ROCm GPU"):
        dec.merge_partial_sets([((m, l, acc), 1, 1)], 4, 1)
    with pytest.raises(ValueError, match="partial sets"):
        dec.merge_partial_sets([((m, l, acc), 1, 1)] * 5, 4, 1)
