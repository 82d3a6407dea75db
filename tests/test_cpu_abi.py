"""The C ABI without a GPU: libava_amd.so loads and exports every entry point include/ava.h declares,
argument errors come back as status codes with a message, and the host-side mirror (ava_amd.ops /
ava_amd.model) refuses CPU tensors instead of falling back to anything."""
import ctypes as C
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def lib():
    from ava_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        from ava_amd import build
        build.build()
    return _lib.lib()


def declared():
    hdr = open(os.path.join(ROOT, "include", "ava.h")).read()
    hdr = re.sub(r"/\*.*?\*/", "", hdr, flags=re.S)
    return sorted(set(re.findall(r"\b(ava_[a-z0-9_]+)\s*\(", hdr)))


def test_header_entry_points_are_exported():
    L = lib()
    names = declared()
    assert len(names) >= 18
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def test_argument_errors_return_status_and_message():
    L = lib()
    assert L.ava_version().startswith(b"ava_amd")
    rc = L.ava_lif_scan(None, 1, 1, 1, None, None, None, None, 2, 1, 1, None, None, None)
    assert rc == 1 and b"NULL" in L.ava_last_error()
    rc = L.ava_mem_scan(None, None, None, None, None, None, 1, 1, 32, 1, C.c_float(0.0), C.c_float(1e5), None,
                        None, None, None)
    assert rc == 4 and b"head size" in L.ava_last_error()
    assert L.ava_q8_ldk(1) == 128 and L.ava_q8_ldk(1024) == 1024 and L.ava_q8_ldk(1025) == 1152


def test_ops_refuse_host_tensors():
    import torch
    from ava_amd import ops
    with pytest.raises(ValueError):
        ops.kwta_relu(torch.zeros((2, 8)), 2)
    with pytest.raises(ValueError):
        ops.lif_gen(torch.zeros((1, 2, 8)), torch.zeros(8))


def test_attend_heads_argument_errors():
    """The heads read refuses NULL buffers and head geometries it does not run before touching the GPU;
    its partials size follows (heads x (hd + 2)) floats per row and chunk."""
    L = lib()
    vp = C.c_void_p
    rc = L.ava_attend_heads(None, 128, None, None, 0, 8, 0, 1, 1, 128, 4, None, None, 0, None)
    assert rc == 1 and b"NULL" in L.ava_last_error()
    dummy = vp(64)  # never dereferenced: the shape checks come first
    for de, heads in ((96, 3), (128, 3), (256, 2), (128, 0)):
        rc = L.ava_attend_heads(dummy, de, dummy, dummy, 0, 8, 0, 1, 1, de, heads, dummy, dummy, 0, None)
        assert rc == 2 and b"heads" in L.ava_last_error(), (de, heads)
    assert L.ava_attend_heads_part_floats(2, 1, 1500, 1024, 32) == 2 * 1 * 32 * 2 * 34
    assert L.ava_attend_heads_part_floats(2, 1, 1500, 64, 1) == L.ava_attend_part_floats(2, 1, 1500) == 2 * 2 * 66
    assert L.ava_attend_heads_part_floats(2, 8, 1500, 1024, 32) == 0  # the tiled form needs none
