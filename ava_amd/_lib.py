"""Loader of the in-tree libava_amd.so and the ctypes signatures of include/ava.h.

The product path has no fallback: if the HIP library is missing, every op raises.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libava_amd.so")

vp = C.c_void_p
i32 = C.c_int
f32 = C.c_float
sz = C.c_size_t


class QW(C.Structure):
    """ava_qw: one int8 weight matrix (device pointers)."""
    _fields_ = [("din", i32), ("dout", i32), ("ldk", i32), ("qt", vp), ("scale", vp)]


class Config(C.Structure):
    _fields_ = [(n, i32) for n in ("vocab", "d", "layers", "hidden", "kwta_k", "head_size", "gate_rank",
                                   "eng_block", "eng_dim", "levels", "alif", "lif_scale", "value_residual",
                                   "dense", "relu2")] + \
               [("momentum", f32), ("cap", f32), ("planes", i32), ("cb_units", i32), ("cb_lr", f32), ("cb_half", f32),
                ("eng_half", i32), ("eng_heads", i32)]


BLOCK_FIELDS = ["lif_norm", "win", "beta_p", "theta", "arho", "again", "wout",
                "mem_norm", "wq", "wk", "wv", "we", "wg", "wo",
                "wa", "ba", "wb", "bb", "off", "wa1", "wa2", "wb1", "wb2", "vres",
                "eng_norm", "ewq", "ewk", "ewv", "ewo",
                "mlp_norm", "w1", "w2", "dense"]


def config_struct(c: dict, planes: int = 3, cb_lr: float = 0.0) -> Config:
    """ava_config from a configuration dict (ava_amd.synth's keys)."""
    return Config(vocab=c["vocab"], d=c["d"], layers=c["layers"], hidden=c["hidden"], kwta_k=c["kwta_k"],
                  head_size=c["head_size"], gate_rank=c["gate_rank"], eng_block=c["eng_block"],
                  eng_dim=c["eng_dim"], levels=c["levels"], alif=int(c["alif"]), lif_scale=int(c["lif_scale"]),
                  value_residual=int(c["value_residual"]), dense=int(c["dense"]), relu2=int(c["relu2"]),
                  momentum=c["momentum"], cap=c["cap"], planes=planes, cb_units=c.get("cb_units", 0),
                  cb_lr=float(cb_lr), cb_half=float(c.get("cb_half", 0.0) or 0.0),
                  eng_half=int(bool(c.get("eng_half", False))), eng_heads=int(c.get("eng_heads", 1) or 1))


class BlockParams(C.Structure):
    _fields_ = [(n, vp) for n in BLOCK_FIELDS]


class Params(C.Structure):
    _fields_ = [("tok_emb", vp), ("final_norm", vp), ("blocks", C.POINTER(BlockParams)), ("cb_w", vp)]


class State(C.Structure):
    _fields_ = [("lif_v", vp), ("lif_s", vp), ("lif_a", vp), ("mem_f", vp), ("mem_s", vp),
                ("eng_k", vp), ("eng_v", vp), ("eng_cap", i32), ("eng_len", i32),
                ("cb_tab", vp), ("cb_scale", vp), ("cb_code", vp), ("eng_len_dev", vp), ("eng_reads", vp),
                ("eng_age", vp)]


_lib = None


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"libava_amd.so is not built ({LIB_PATH}); run `python -m ava_amd.build`")
    L = C.CDLL(LIB_PATH)
    L.ava_last_error.restype = C.c_char_p
    L.ava_version.restype = C.c_char_p
    L.ava_fnv1a64.argtypes = [vp, sz, C.c_uint64]
    L.ava_fnv1a64.restype = C.c_uint64
    sig = {
        "ava_q8_ldk": [i32],
        "ava_q8_pack": [vp, i32, i32, vp, vp, vp],
        "ava_q8_quant_rows": [vp, i32, i32, i32, vp, vp, vp],
        "ava_q8_gemm_acc": [vp, i32, i32, C.POINTER(QW), vp, vp],
        "ava_q8_matmul": [vp, i32, C.POINTER(QW), i32, vp, vp, sz, vp],
        "ava_q8_matmul_i8": [vp, i32, C.POINTER(QW), vp, vp],
        "ava_q8_matmul_noalloc": [vp, i32, C.POINTER(QW), i32, vp, vp],
        "ava_q8_matmul_planes": [vp, vp, i32, i32, C.POINTER(QW), vp, vp],
        "ava_lif_scan": [vp, i32, i32, i32, vp, vp, vp, vp, i32, i32, i32, vp, vp, vp],
        "ava_kwta": [vp, i32, i32, i32, i32, vp, vp, vp],
        "ava_mem_scan": [vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, f32, f32, vp, vp, vp, vp],
        "ava_mem_chunk": [vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, f32, f32, vp, vp, vp, vp],
        "ava_delta_chunk": [vp, vp, vp, vp, vp, i32, i32, i32, vp, vp, vp, sz, vp],
        "ava_lif_scan_bwd": [vp, i32, i32, i32, vp, vp, vp, vp, i32, i32, i32, f32, i32] + [vp] * 10,
        "ava_lif_scan_bwd_segments": [vp, i32, i32, i32, vp, vp, vp, vp, i32, i32, i32, f32, i32] + [vp] * 10 + [sz, vp],
        "ava_kwta_relu2_bwd": [vp, vp, i32, i32, vp, vp, vp],
        "ava_mem_scan_bwd": [vp] * 6 + [i32] * 4 + [f32, f32] + [vp] * 14 + [sz, vp],
        "ava_dense_back": [vp] * 6 + [i32] * 4 + [C.c_longlong, vp, sz, vp],
        "ava_attend": [vp, i32, vp, vp, i32, i32, i32, i32, i32, vp, vp, sz, vp],
        "ava_attend_heads": [vp, i32, vp, vp, i32, i32, i32, i32, i32, i32, i32, vp, vp, sz, vp],
        "ava_model_new": [C.POINTER(Config), C.POINTER(Params), C.POINTER(vp)],
        "ava_model_forward": [vp, C.POINTER(State), vp, i32, i32, vp, vp],
        "ava_model_cb_learn": [vp, C.POINTER(State), vp, i32, vp, i32, vp, vp],
        "ava_model_decode_step": [vp, C.POINTER(State), vp, i32, i32, vp, vp, i32, vp, vp, vp],
        "ava_engram_evict": [vp, vp, vp, vp, i32, i32, i32, vp, i32, i32, i32, i32, vp],
        "ava_train_new": [C.POINTER(Config), f32, i32, C.POINTER(vp)],
        "ava_train_param_slot": [vp, C.c_char_p, i32, C.POINTER(sz), C.POINTER(sz)],
        "ava_train_step": [vp, vp, vp, vp, i32, i32, vp, vp, vp],
        "ava_train_decisions": [vp, vp, vp, vp, vp],
    }
    for name, args in sig.items():
        fn = getattr(L, name, None)
        if fn is None:
            continue
        fn.argtypes = args
        fn.restype = i32
    L.ava_attend_part_floats.argtypes = [i32, i32, i32]
    L.ava_attend_part_floats.restype = sz
    L.ava_attend_heads_part_floats.argtypes = [i32, i32, i32, i32, i32]
    L.ava_attend_heads_part_floats.restype = sz
    L.ava_mem_scan_bwd_workspace.argtypes = [i32, i32, i32]
    L.ava_mem_scan_bwd_workspace.restype = sz
    L.ava_delta_chunk_workspace.argtypes = [i32, i32]
    L.ava_delta_chunk_workspace.restype = sz
    L.ava_lif_scan_bwd_segments_workspace.argtypes = [i32, i32, i32]
    L.ava_lif_scan_bwd_segments_workspace.restype = sz
    L.ava_dense_back_part_floats.argtypes = [C.c_longlong, i32]
    L.ava_dense_back_part_floats.restype = sz
    L.ava_train_free.argtypes = [vp]
    L.ava_train_free.restype = None
    L.ava_train_param_floats.argtypes = [vp]
    L.ava_train_param_floats.restype = sz
    L.ava_q8_workspace.argtypes = [i32, i32, i32]
    L.ava_q8_workspace.restype = sz
    if hasattr(L, "ava_model_free"):
        L.ava_model_free.argtypes = [vp]
        L.ava_model_free.restype = None
    if hasattr(L, "ava_model_freeze"):
        L.ava_model_freeze.argtypes = [vp, i32]
        L.ava_model_freeze.restype = i32
    if hasattr(L, "ava_model_scratch_bytes"):
        L.ava_model_scratch_bytes.argtypes = [vp]
        L.ava_model_scratch_bytes.restype = sz
    L.ava_model_nonfinite.argtypes = [vp, vp, i32, C.POINTER(C.c_int), vp]
    L.ava_model_nonfinite.restype = i32
    L.ava_model_set_trace.argtypes = [vp, vp, vp, vp, sz]
    L.ava_model_set_trace.restype = i32
    if hasattr(L, "ava_model_set_timing"):
        L.ava_model_set_timing.argtypes = [vp, i32]
        L.ava_model_set_timing.restype = i32
        L.ava_model_timing.argtypes = [vp, C.POINTER(C.c_char_p), C.POINTER(C.c_int), C.POINTER(C.c_double), i32, i32]
        L.ava_model_timing.restype = i32
    _lib = L
    return L


class AvaError(RuntimeError):
    pass


def check(rc: int, what: str = ""):
    if rc != 0:
        msg = lib().ava_last_error().decode(errors="replace")
        raise AvaError(f"{what or 'ava'} failed ({rc}): {msg}")
