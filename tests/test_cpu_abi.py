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
    n = C.c_int(7)
    rows = (C.c_int32 * 4)()
    assert L.ava_model_nonfinite(None, rows, 4, C.byref(n), None) == 1 and b"NULL" in L.ava_last_error()
    # the training step refuses what it does not build before touching the GPU
    from ava_amd import synth
    from ava_amd._lib import config_struct
    h = C.c_void_p()
    assert L.ava_train_new(None, C.c_float(4.0), 0, C.byref(h)) == 1
    bad = synth.config("tiny")
    bad["head_size"] = 32
    assert L.ava_train_new(C.byref(config_struct(bad)), C.c_float(4.0), 0, C.byref(h)) == 2
    assert b"head size 64" in L.ava_last_error() and not h.value
    cb = synth.config("tiny_cb")
    assert L.ava_train_new(C.byref(config_struct(cb)), C.c_float(4.0), 0, C.byref(h)) == 1


def test_scan_and_product_argument_errors():
    """The segmented LIF backward refuses a short workspace and a bad level count, the product a plane
    count outside 1..3, a short workspace and weights whose K padding is wrong, all before touching the
    GPU (the pointers below are never dereferenced)."""
    from ava_amd._lib import QW
    L = lib()
    d = C.c_void_p(64)
    B, T, D = 2, 100, 64
    need = L.ava_lif_scan_bwd_segments_workspace(B, T, D)
    assert need > 0 and L.ava_lif_scan_bwd_segments_workspace(0, T, D) == 0
    args = lambda levels, ws_bytes: (d, B, T, D, d, d, d, d, levels, 1, 1, C.c_float(1.0), 1, d, d, d, d, d, d, d, d,
                                     d, d, ws_bytes, None)
    assert L.ava_lif_scan_bwd_segments(*args(2, need - 4)) == 2 and b"workspace" in L.ava_last_error()
    assert L.ava_lif_scan_bwd_segments(*args(3, need)) == 1 and b"levels" in L.ava_last_error()
    w = QW(din=100, dout=8, ldk=L.ava_q8_ldk(100), qt=64, scale=64)
    ws = L.ava_q8_workspace(10, 100, 3)
    assert L.ava_q8_matmul(d, 10, C.byref(w), 4, d, d, ws, None) == 1 and b"planes" in L.ava_last_error()
    assert L.ava_q8_matmul(d, 10, C.byref(w), 3, d, d, ws - 1, None) == 2 and b"workspace" in L.ava_last_error()
    bad = QW(din=100, dout=8, ldk=100, qt=64, scale=64)
    assert L.ava_q8_matmul(d, 10, C.byref(bad), 3, d, d, ws, None) == 2 and b"ldk" in L.ava_last_error()
    assert L.ava_q8_matmul(d, 0, C.byref(w), 3, d, d, ws, None) == 0  # no rows: nothing to do


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


# ----------------------------------------------------------------------------- the binding guide vs the header

_C_WIDTH = {"int": "i32", "float": "f32", "double": "f64", "size_t": "usize", "uint64_t": "u64"}
_RS_WIDTH = {"c_int": "i32", "i32": "i32", "c_float": "f32", "f32": "f32", "c_double": "f64", "f64": "f64",
             "usize": "usize", "u64": "u64"}


def header_structs():
    """{struct name: [(field, width)]} of include/ava.h's typedef structs; pointers are 'ptr'."""
    hdr = open(os.path.join(ROOT, "include", "ava.h")).read()
    hdr = re.sub(r"/\*.*?\*/", "", hdr, flags=re.S)
    out = {}
    for body, name in re.findall(r"typedef struct\s*\{(.*?)\}\s*(\w+)\s*;", hdr, flags=re.S):
        fields = []
        for decl in body.split(";"):
            decl = " ".join(decl.split())
            if not decl:
                continue
            m = re.match(r"((?:const\s+)?\w+)\s+(.*)", decl)
            base, rest = m.group(1).replace("const ", ""), m.group(2)
            for dcl in rest.split(","):
                dcl = dcl.strip()
                ptr = dcl.startswith("*")
                fields.append((dcl.lstrip("*").strip(), "ptr" if ptr else _C_WIDTH[base]))
        out[name] = fields
    return out


def header_functions():
    """{function name: number of parameters} of include/ava.h."""
    hdr = open(os.path.join(ROOT, "include", "ava.h")).read()
    hdr = re.sub(r"/\*.*?\*/", "", hdr, flags=re.S)
    out = {}
    for name, args in re.findall(r"\b(ava_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", hdr):
        args = args.strip()
        out[name] = 0 if args in ("", "void") else len(args.split(","))
    return out


def guide_rust():
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    return text[text.index("```rust"):text.index("```", text.index("```rust") + 7)]


def guide_structs():
    out = {}
    for name, body in re.findall(r"#\[repr\(C\)\]\s*pub struct (\w+)\s*\{(.*?)\n?\}", guide_rust(), flags=re.S):
        body = re.sub(r"//[^\n]*", "", body)
        fields = []
        for name_, ty in re.findall(r"pub (\w+):\s*([^,]+?)\s*(?:,|$)", body.strip()):
            ty = ty.strip()
            fields.append((name_, "ptr" if ty.startswith("*") else _RS_WIDTH[ty]))
        if fields:
            out[name] = fields
    return out


def guide_functions():
    block = guide_rust()
    block = block[block.index('extern "C"'):]
    out = {}
    for name, args in re.findall(r"pub fn (ava_\w+)\s*\(([^)]*)\)", block, flags=re.S):
        args = args.strip().rstrip(",")
        out[name] = 0 if not args else len(args.split(","))
    return out


def test_binding_guide_structs_match_the_header():
    """The binding guide's #[repr(C)] structs have the header's fields in the header's order and widths,
    so a binding written from the guide passes structs of the right size and layout."""
    hs, gs = header_structs(), guide_structs()
    for name in ("ava_qw", "ava_config", "ava_block_params", "ava_params", "ava_state"):
        assert name in hs and name in gs, name
        assert gs[name] == hs[name], (name, [a for a, b in zip(gs[name], hs[name]) if a != b] or
                                      (len(gs[name]), len(hs[name])))


def test_binding_guide_declares_every_entry_point():
    """Every function of include/ava.h is in the guide's extern block with the same number of arguments."""
    hf, gf = header_functions(), guide_functions()
    assert set(hf) == set(declared())
    missing = sorted(set(hf) - set(gf))
    assert not missing, missing
    wrong = {n: (gf[n], hf[n]) for n in hf if gf[n] != hf[n]}
    assert not wrong, wrong


def test_ctypes_structs_match_the_header():
    """ava_amd/_lib.py's ctypes structs have the header's field order and widths."""
    from ava_amd import _lib
    width = {C.c_int: "i32", C.c_float: "f32", C.c_double: "f64", C.c_size_t: "usize", C.c_uint64: "u64"}

    def fields(cls):
        out = []
        for name, ty in cls._fields_:
            if ty in width:
                out.append((name, width[ty]))
            else:
                assert ty is C.c_void_p or issubclass(ty, C._Pointer), (cls, name, ty)
                out.append((name, "ptr"))
        return out

    hs = header_structs()
    pairs = {"ava_qw": _lib.QW, "ava_config": _lib.Config, "ava_block_params": _lib.BlockParams,
             "ava_params": _lib.Params, "ava_state": _lib.State}
    for name, cls in pairs.items():
        assert fields(cls) == hs[name], name


def test_ctypes_signatures_match_the_header():
    """Every entry point that ava_amd/_lib.py gives argtypes takes the header's number of parameters,
    so a ctypes call can never shift its arguments."""
    L = lib()
    hf = header_functions()
    wrong = {}
    for name, n in hf.items():
        fn = getattr(L, name)
        if fn.argtypes is not None and len(fn.argtypes) != n:
            wrong[name] = (len(fn.argtypes), n)
    assert not wrong, wrong
