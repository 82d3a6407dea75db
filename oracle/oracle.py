"""ctypes front of the CPU oracle (oracle/libava_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, always as the checker, never as the thing measured on the GPU path.
Each wrapper names the C function (and through it the reference file:line) it calls.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = os.path.join(_HERE, "libava_oracle.so")
_lib = None

f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
i8p = np.ctypeslib.ndpointer(dtype=np.int8, flags="C_CONTIGUOUS")
i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (gcc; no GPU needed)."""
    if force or not os.path.exists(_LIB):
        subprocess.run(["make", "-s", "-B" if force else "all"], cwd=_HERE, check=True)
    return _LIB


def lib():
    global _lib
    if _lib is None:
        build()
        L = C.CDLL(_LIB)
        L.orc_quantize_int8.argtypes = [f32p, C.c_int, C.c_int, i8p, f32p]
        L.orc_q8_matmul_ref.argtypes = [f32p, C.c_int, C.c_int, i8p, f32p, C.c_int, f32p, C.c_int]
        L.orc_q8_matmul_rows.argtypes = L.orc_q8_matmul_ref.argtypes
        L.orc_q8_matmul_blocked.argtypes = L.orc_q8_matmul_ref.argtypes
        L.orc_quant_planes.argtypes = [f32p, C.c_int, C.c_int, C.c_int, i8p, i32p]
        L.orc_q8_acc.argtypes = [i8p, C.c_int, C.c_int, i8p, C.c_int, i32p, C.c_int]
        L.orc_q8_combine.argtypes = [i32p, C.c_int, C.c_void_p, C.c_int, f32p, C.c_int, f32p]
        L.orc_q8_matmul_planes.argtypes = [f32p, C.c_int, C.c_int, C.c_int, i8p, f32p, C.c_int, f32p, C.c_int]
        L.orc_lif_scan.argtypes = [f32p, C.c_int, C.c_int, C.c_int, f32p, f32p, f32p, f32p,
                                   C.c_int, C.c_int, C.c_int, i8p]
        L.orc_kwta.argtypes = [f32p, C.c_int, C.c_int, C.c_int, C.c_int, f32p, f32p]
        L.orc_mem_rec.argtypes = [f32p] * 6 + [C.c_int] * 4 + [C.c_float, C.c_float, f32p, C.c_void_p, f32p]
        L.orc_mem_chunk.argtypes = [f32p] * 6 + [C.c_int] * 4 + [C.c_float, f32p, C.c_void_p, f32p]
        L.orc_set_mem_chunked.argtypes = [C.c_int]
        L.orc_set_mem_chunked.restype = None
        L.orc_mem_rec_f64.argtypes = [f32p] * 6 + [C.c_int] * 4 + [C.c_double, f64p, C.c_void_p, f64p]
        L.orc_mem_rec_f64d.argtypes = [f64p] * 6 + [C.c_int] * 3 + [C.c_double, C.c_double, f64p, C.c_void_p, f64p]
        L.orc_rmsnorm.argtypes = [f32p, C.c_int, C.c_int, f32p, f32p]
        L.orc_round_half.argtypes = [C.c_float]
        L.orc_round_half.restype = C.c_float
        L.orc_sigmoid.argtypes = [C.c_float]
        L.orc_sigmoid.restype = C.c_float
        L.orc_log_sigmoid.argtypes = [C.c_float]
        L.orc_log_sigmoid.restype = C.c_float
        L.orc_cb_wiring.argtypes = [C.c_int, C.c_int, C.c_int, C.c_uint64, C.c_void_p, C.c_void_p]
        L.orc_cb_code.argtypes = [f32p, f32p, C.c_int, C.c_void_p, f32p, C.c_int, C.c_int, C.c_int, f32p]
        L.orc_cb_apply.argtypes = [f32p, f32p, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_double, f32p]
        L.orc_cb_learn.restype = C.c_double
        L.orc_cb_learn.argtypes = [f32p, C.c_int, C.c_int, f32p, C.c_int, f32p, C.c_int, C.c_float, C.c_double,
                                   C.POINTER(C.c_double), f32p]
        L.orc_lif_bwd.argtypes = ([f32p, C.c_int, C.c_int, C.c_int, f32p, f32p, f32p, f32p, C.c_int, C.c_int, C.c_int,
                                   C.c_float, C.c_int, f32p, C.c_void_p, C.c_void_p] + [f32p] * 6)
        L.orc_mem_rec_bwd.argtypes = ([f32p] * 6 + [C.c_int] * 4 + [C.c_float, C.c_float] + [C.c_void_p] * 2 +
                                      [f32p] + [C.c_void_p] * 2 + [f32p] * 6 + [C.c_void_p] * 2)
        L.orc_set_threads.argtypes = [C.c_int]
        L.orc_set_threads.restype = None
        L.orc_model_forward.restype = C.c_int
        L.orc_model_forward.argtypes = [C.POINTER(_Cfg), C.POINTER(_Model), C.c_void_p, C.c_int, C.c_int,
                                        C.POINTER(_State), C.c_void_p, C.c_int, C.c_int, C.POINTER(_Trace)]
        _lib = L
    return _lib


def set_threads(n: int):
    """The thread count of the oracle's parallel loops over rows, channels and heads (the same bits
    at any count)."""
    lib().orc_set_threads(int(n))


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


# --------------------------------------------------------------------------- int8 products

def quantize_int8(w):
    """parts/src/quant.rs:18-31 -> (q int8 [din, dout], scale f32 [dout])."""
    w = _c(w, np.float32)
    din, dout = w.shape
    q = np.empty((din, dout), np.int8)
    s = np.empty(dout, np.float32)
    lib().orc_quantize_int8(w, din, dout, q, s)
    return q, s


def q8_matmul_ref(x, q, scale, threads=1, form="auto"):
    """gpu/int8.rs:301-331: W8A32, f32 fma chain in j order, times the column scale. form: "rows" (the
    per-row kernel), "blocked" (gpu/int8/block.rs's 6 x 16 register blocks) or "auto" (blocked from 6
    rows, as the reference chooses); the same bits every way."""
    x = _c(x, np.float32)
    m, din = x.shape
    dout = q.shape[1]
    y = np.empty((m, dout), np.float32)
    fn = {"auto": lib().orc_q8_matmul_ref, "rows": lib().orc_q8_matmul_rows, "blocked": lib().orc_q8_matmul_blocked}[form]
    fn(x, m, din, _c(q, np.int8), _c(scale, np.float32), dout, y, threads)
    return y


def quant_planes(x, planes):
    x = _c(x, np.float32)
    m, k = x.shape
    xq = np.empty((planes, m, k), np.int8)
    xe = np.empty(m, np.int32)
    lib().orc_quant_planes(x, m, k, planes, xq, xe)
    return xq, xe


def q8_acc(a, q, threads=1):
    a = _c(a, np.int8)
    m, k = a.shape
    n = q.shape[1]
    acc = np.empty((m, n), np.int32)
    lib().orc_q8_acc(a, m, k, _c(q, np.int8), n, acc, threads)
    return acc


def q8_combine(acc, xexp, scale):
    acc = _c(acc, np.int32)
    planes, m, n = acc.shape
    y = np.empty((m, n), np.float32)
    xe = None if xexp is None else _c(xexp, np.int32)
    lib().orc_q8_combine(acc, planes, None if xe is None else xe.ctypes.data, m, _c(scale, np.float32), n, y)
    return y


def q8_matmul_planes(x, planes, q, scale, threads=1):
    x = _c(x, np.float32)
    m, k = x.shape
    n = q.shape[1]
    y = np.empty((m, n), np.float32)
    lib().orc_q8_matmul_planes(x, m, k, planes, _c(q, np.int8), _c(scale, np.float32), n, y, threads)
    return y


# --------------------------------------------------------------------------- LIF, kWTA, memory

def lif_scan(cur, ps, v0=None, s0=None, a0=None, levels=2, signed=True, alif=True):
    """gpu/lif_gen.rs:151-214. cur [B, T, D]; ps [4D] = beta|theta|rho|gain.
    Returns (spikes int8 [B, T, D], v [B, D], s [B, D], a [B, D])."""
    cur = _c(cur, np.float32)
    B, T, D = cur.shape
    v = np.zeros((B, D), np.float32) if v0 is None else _c(v0, np.float32).copy()
    s = np.zeros((B, D), np.float32) if s0 is None else _c(s0, np.float32).copy()
    a = np.zeros((B, D), np.float32) if a0 is None else _c(a0, np.float32).copy()
    spk = np.empty((B, T, D), np.int8)
    lib().orc_lif_scan(cur, B, T, D, _c(ps, np.float32), v, s, a, levels, int(signed), int(alif), spk)
    return spk, v, s, a


def round_half(x):
    """IEEE binary16 round-to-nearest-even of each element (the oracle's orc_round_half), as float32."""
    f = np.vectorize(lambda v: lib().orc_round_half(float(v)), otypes=[np.float32])
    return f(np.asarray(x, np.float32))


def lif_params(block, alif=True):
    """The scan's per-channel parameters of one block as the oracle's forward forms them
    (ava_oracle.c, after gpu/arch.rs:1632-1695): beta = sigmoid(beta_p) | theta | rho = sigmoid(arho)
    | gain, in f32 with the oracle's own sigmoid."""
    f = np.vectorize(lambda x: lib().orc_sigmoid(float(x)), otypes=[np.float32])
    z = np.zeros_like(block["theta"], dtype=np.float32)
    return np.concatenate([f(block["beta_p"]), np.asarray(block["theta"], np.float32),
                           f(block["arho"]) if alif else z, np.asarray(block["again"], np.float32) if alif else z])


def kwta(u, k, relu2=True):
    """gpu/model/fstep.rs:295-299 + fstep/arch.rs:976-989 -> (a [n, h], kth [n])."""
    u = _c(u, np.float32)
    n, h = u.shape
    a = np.empty((n, h), np.float32)
    kth = np.empty(n, np.float32)
    lib().orc_kwta(u, n, h, k, int(relu2), a, kth)
    return a, kth


def mem_rec(q, k, e, v, la, b, m=0.0, cap=1e5, F=None, S=None):
    """gpu/mem_gen.rs:220-273. q, k, e, v [BH, T, hs]; la, b [BH, T, g]. Returns (y, F, S)."""
    q, k, e, v, la, b = (_c(z, np.float32) for z in (q, k, e, v, la, b))
    BH, T, hs = q.shape
    g = la.shape[2]
    F = np.zeros((BH, hs, hs), np.float32) if F is None else _c(F, np.float32).copy()
    S = np.zeros((BH, hs, hs), np.float32) if S is None else _c(S, np.float32).copy()
    y = np.empty((BH, T, hs), np.float32)
    lib().orc_mem_rec(q, k, e, v, la, b, BH, T, hs, g, float(m), float(cap), F,
                      S.ctypes.data if m != 0.0 else None, y)
    return y, F, S


def mem_chunk(q, k, e, v, la, b, m=0.0, F=None, S=None):
    """gpu/arch.rs:1151-1164, 1243-1327 (delta_chunk): mem_rec's rule in chunks, no bound. Returns (y, F, S)."""
    q, k, e, v, la, b = (_c(z, np.float32) for z in (q, k, e, v, la, b))
    BH, T, hs = q.shape
    g = la.shape[2]
    F = np.zeros((BH, hs, hs), np.float32) if F is None else _c(F, np.float32).copy()
    S = np.zeros((BH, hs, hs), np.float32) if S is None else _c(S, np.float32).copy()
    y = np.empty((BH, T, hs), np.float32)
    lib().orc_mem_chunk(q, k, e, v, la, b, BH, T, hs, g, float(m), F, S.ctypes.data if m != 0.0 else None, y)
    return y, F, S


def evict_engram(state, eng_max, rule="oldest"):
    """gpu/state.rs:518-590 (evict): when a stream's store holds more than eng_max slots, keep eng_max.
    oldest: the last eng_max. least-read (needs the state's counts): rank every slot by (class, value,
    index), class 1 for a slot some later query could see (age >= 1; value = reads / age, the mean mass
    per later query) and class 2 for the slots no later query has seen yet (value 0); keep the last
    eng_max of the ranking, in store order. The store, counts and length are updated in place. The ranking is written out as plain
    Python sorts over (class, value, index) tuples, as the reference's sort_by."""
    n = state["eng_len"]
    if not eng_max or n <= eng_max:
        return
    B = state["eng_k"].shape[0]
    if rule == "oldest" or "eng_reads" not in state:
        keeps = [list(range(n - eng_max, n))] * B
    else:
        keeps = []
        for r in range(B):
            reads, age = state["eng_reads"][r], state["eng_age"][r]
            order = []
            for j in range(n):
                if age[j] >= 1.0:
                    order.append((1, float(np.float32(reads[j]) / np.float32(age[j])), j))
                else:
                    order.append((2, 0.0, j))
            order.sort()
            keeps.append(sorted(j for _, _, j in order[n - eng_max:]))
    for r in range(B):
        idx = np.asarray(keeps[r], np.int64)
        for key in ("eng_k", "eng_v"):
            state[key][r, :eng_max] = state[key][r, idx].copy()
        for key in ("eng_reads", "eng_age"):
            if key in state:
                state[key][r, :eng_max] = state[key][r, idx].copy()
    state["eng_len"] = eng_max


def set_mem_chunked(on: bool):
    """The block stack's memory form for T > 1: chunked (the reference's default) or the token loop."""
    lib().orc_set_mem_chunked(int(bool(on)))


def mem_rec_f64d(q, k, e, v, al, b, m=0.0, cap=np.inf):
    """The bounded rule in float64 from a zero state: float64 inputs [BH, T, hs] (al = alpha per channel).
    Returns (y, F, S) float64 (S zeros without momentum)."""
    q, k, e, v, al, b = (_c(z, np.float64) for z in (q, k, e, v, al, b))
    BH, T, hs = q.shape
    F = np.zeros((BH, hs, hs), np.float64)
    S = np.zeros((BH, hs, hs), np.float64)
    y = np.empty((BH, T, hs), np.float64)
    lib().orc_mem_rec_f64d(q, k, e, v, al, b, BH, T, hs, float(m), float(cap), F,
                           S.ctypes.data if m != 0.0 else None, y)
    return y, F, S


def mem_rec_f64(q, k, e, v, la, b, m=0.0, F=None, S=None):
    q, k, e, v, la, b = (_c(z, np.float32) for z in (q, k, e, v, la, b))
    BH, T, hs = q.shape
    g = la.shape[2]
    F = np.zeros((BH, hs, hs), np.float64) if F is None else _c(F, np.float64).copy()
    S = np.zeros((BH, hs, hs), np.float64) if S is None else _c(S, np.float64).copy()
    y = np.empty((BH, T, hs), np.float64)
    lib().orc_mem_rec_f64(q, k, e, v, la, b, BH, T, hs, g, float(m), F,
                          S.ctypes.data if m != 0.0 else None, y)
    return y, F, S


# --------------------------------------------------------------------------- backward (training)

def _ptr(a):
    return None if a is None else a.ctypes.data


def lif_bwd(cur, ps, g_spk, v0=None, s0=None, a0=None, g_vT=None, g_aT=None, levels=2, signed=True, alif=True,
            slope=1.0, reset_grad=False):
    """The LIF scan's backward (orc_lif_bwd: gpu/arch.rs:964-1071 lif_ref's surrogate gradient,
    gpu/lif.cu:3228-3290). Returns dict dI [B, T, D], dv0, da0, dbeta, drho, dgain [B, D]."""
    cur, g_spk = _c(cur, np.float32), _c(g_spk, np.float32)
    B, T, D = cur.shape
    z = np.zeros((B, D), np.float32)
    v0, s0, a0 = (z if x is None else _c(x, np.float32) for x in (v0, s0, a0))
    g_vT = None if g_vT is None else _c(g_vT, np.float32)
    g_aT = None if g_aT is None else _c(g_aT, np.float32)
    out = {k: np.empty((B, D), np.float32) for k in ("dv0", "da0", "dbeta", "drho", "dgain")}
    dI = np.empty((B, T, D), np.float32)
    lib().orc_lif_bwd(cur, B, T, D, _c(ps, np.float32), v0, s0, a0, levels, int(signed), int(alif), float(slope),
                      int(reset_grad), g_spk, _ptr(g_vT), _ptr(g_aT), dI, out["dv0"], out["da0"], out["dbeta"],
                      out["drho"], out["dgain"])
    out["dI"] = dI
    return out


def mem_rec_bwd(q, k, e, v, la, b, dy, m=0.0, cap=1e5, F0=None, S0=None, dF_T=None, dS_T=None):
    """The fast-weight recurrence's backward (orc_mem_rec_bwd: delta_rec's gradient, gpu/arch.rs:1091-1136),
    float64 inside. Returns dict dq, dk, de, dv [BH, T, hs], dla, db [BH, T, g], dF0, dS0 [BH, hs, hs]."""
    q, k, e, v, la, b, dy = (_c(x, np.float32) for x in (q, k, e, v, la, b, dy))
    BH, T, hs = q.shape
    g = la.shape[2]
    F0, S0, dF_T, dS_T = (None if x is None else _c(x, np.float32) for x in (F0, S0, dF_T, dS_T))
    o = {n: np.empty((BH, T, hs), np.float32) for n in ("dq", "dk", "de", "dv")}
    o.update({n: np.empty((BH, T, g), np.float32) for n in ("dla", "db")})
    o["dF0"] = np.empty((BH, hs, hs), np.float32)
    o["dS0"] = np.zeros((BH, hs, hs), np.float32)
    lib().orc_mem_rec_bwd(q, k, e, v, la, b, BH, T, hs, g, float(m), float(cap), _ptr(F0), _ptr(S0), dy, _ptr(dF_T),
                          _ptr(dS_T), o["dq"], o["dk"], o["de"], o["dv"], o["dla"], o["db"], _ptr(o["dF0"]),
                          _ptr(o["dS0"]))
    return o


def kwta_relu2_bwd(u, kth, ga):
    """The backward of relu² after kWTA (gpu/lif.cu:4666-4679 relu2_bwd; the mask of gpu/lif.cu:4647):
    gu = (u ga) 2 where u - kth >= 0 and u > 0, else 0; each product rounded alone, in f32."""
    u, ga = _c(u, np.float32), _c(ga, np.float32)
    kth = _c(kth, np.float32)[:, None]
    keep = (u - kth >= 0) & (u > 0)
    return np.where(keep, (u * ga).astype(np.float32) * np.float32(2), np.float32(0)).astype(np.float32)


def dense_back(S, G, wf, base, col, i0, L, nd):
    """The dense mix's backward (gpu/lif.cu:4922-4971 dense_back, the mix of gpu/arch.rs:1492-1500):
    out = base + sum_{k=i0..L-1} w_k[col] G_k (added in k order, f32), dw[j] = sum_e base_e S_j,e
    (float64 here). wf packs block k's k + 2 weights from k (k + 3) / 2."""
    base = _c(base, np.float32)
    out = base.copy()
    for k in range(i0, L):
        out = (out + np.float32(wf[k * (k + 3) // 2 + col]) * np.asarray(G[k], np.float32)).astype(np.float32)
    dw = np.array([np.dot(base.astype(np.float64).ravel(), np.asarray(S[j], np.float64).ravel())
                   for j in range(nd)], np.float64)
    return out, dw


def rmsnorm(x, gain):
    x = _c(x, np.float32)
    n, d = x.shape
    out = np.empty_like(x)
    lib().orc_rmsnorm(x, n, d, _c(gain, np.float32), out)
    return out


def sigmoid(x):
    return np.float32(lib().orc_sigmoid(float(x)))


def log_sigmoid(x):
    return np.float32(lib().orc_log_sigmoid(float(x)))


# --------------------------------------------------------------------------- cerebellum head


def cb_wiring(inputs, g, fan_in, seed):
    """gpu/v51b.rs:242-265: idx [g, fan_in] uint32, sgn [g, fan_in] f32."""
    idx = np.empty((g, fan_in), np.uint32)
    sgn = np.empty((g, fan_in), np.float32)
    lib().orc_cb_wiring(inputs, g, fan_in, C.c_uint64(seed), idx.ctypes.data, sgn.ctypes.data)
    return idx, sgn


def cb_code(xf, emb_row, idx, sgn, k):
    """gpu/model/fstep/arch_f3.rs:225-262: the unit-length granule code c [g] of one row."""
    xf, emb_row = _c(xf, np.float32), _c(emb_row, np.float32)
    idx, sgn = _c(idx, np.uint32), _c(sgn, np.float32)
    g, fan_in = sgn.shape
    c = np.empty(g, np.float32)
    lib().orc_cb_code(xf, emb_row, xf.shape[0], idx.ctypes.data, sgn, g, fan_in, k, c)
    return c


def cb_apply(xf, c, w=None, tab=None, scale=1.0):
    """gpu/model/fstep/arch_f3.rs:262-299 + gpu/v51b.rs:373-389: xf + c.W (+ the table's share)."""
    xf, c = _c(xf, np.float32), _c(c, np.float32)
    w = None if w is None else _c(w, np.float32)
    tab = None if tab is None else _c(tab, np.float32)
    out = np.empty_like(xf)
    lib().orc_cb_apply(xf, c, c.shape[0], xf.shape[0], None if w is None else w.ctypes.data,
                       None if tab is None else tab.ctypes.data, C.c_double(scale), out)
    return out


def cb_learn(logits, nxt, E, c, lr, half, scale, tab):
    """gpu/fast4/cb.rs:25-84: one online step of a stream's table tab [g, d] (updated in place).
    Returns (nats, new scale)."""
    logits, E, c = _c(logits, np.float32), _c(E, np.float32), _c(c, np.float32)
    assert tab.dtype == np.float32 and tab.flags.c_contiguous
    sc = C.c_double(scale)
    nats = lib().orc_cb_learn(logits, logits.shape[0], int(nxt), E, E.shape[1], c, c.shape[0], C.c_float(lr),
                              C.c_double(half if half and half > 0 else 0.0), C.byref(sc), tab)
    return nats, sc.value


# --------------------------------------------------------------------------- model

class _QW(C.Structure):
    _fields_ = [("q", C.c_void_p), ("scale", C.c_void_p), ("din", C.c_int), ("dout", C.c_int)]


_BLOCK_F32 = ["lif_norm", "beta_p", "theta", "arho", "again", "mem_norm", "wa", "ba", "wb", "bb", "off",
              "wa1", "wa2", "wb1", "wb2", "vres", "eng_norm", "mlp_norm", "dense"]
_BLOCK_Q8 = ["win", "wout", "wq", "wk", "wv", "we", "wg", "wo", "ewq", "ewk", "ewv", "ewo", "w1", "w2"]


class _Block(C.Structure):
    _fields_ = [("lif_norm", C.c_void_p), ("win", _QW), ("beta_p", C.c_void_p), ("theta", C.c_void_p),
                ("arho", C.c_void_p), ("again", C.c_void_p), ("wout", _QW), ("mem_norm", C.c_void_p),
                ("wq", _QW), ("wk", _QW), ("wv", _QW), ("we", _QW), ("wg", _QW), ("wo", _QW),
                ("wa", C.c_void_p), ("ba", C.c_void_p), ("wb", C.c_void_p), ("bb", C.c_void_p),
                ("off", C.c_void_p), ("wa1", C.c_void_p), ("wa2", C.c_void_p), ("wb1", C.c_void_p),
                ("wb2", C.c_void_p), ("vres", C.c_void_p), ("eng_norm", C.c_void_p),
                ("ewq", _QW), ("ewk", _QW), ("ewv", _QW), ("ewo", _QW), ("mlp_norm", C.c_void_p),
                ("w1", _QW), ("w2", _QW), ("dense", C.c_void_p)]


class _Cfg(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("vocab", "d", "layers", "hidden", "kwta_k", "heads", "head_size",
                                       "gate_rank", "eng_block", "eng_dim", "levels", "alif", "lif_scale",
                                       "value_residual", "dense", "relu2")] + \
               [("momentum", C.c_float), ("cap", C.c_float), ("eng_half", C.c_int), ("eng_heads", C.c_int)]


class _Model(C.Structure):
    _fields_ = [("tok_emb", C.c_void_p), ("head", _QW), ("final_norm", C.c_void_p), ("blocks", C.POINTER(_Block))]


class _State(C.Structure):
    _fields_ = [("lif_v", C.c_void_p), ("lif_s", C.c_void_p), ("lif_a", C.c_void_p), ("mem_f", C.c_void_p),
                ("mem_s", C.c_void_p), ("eng_k", C.c_void_p), ("eng_v", C.c_void_p), ("eng_cap", C.c_int),
                ("eng_len", C.c_int), ("eng_reads", C.c_void_p), ("eng_age", C.c_void_p)]


class _Trace(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("spikes", "cur", "u", "kth", "memy", "x", "hf", "force_spikes",
                                         "force_keep", "vm", "tht")]


class OracleModel:
    """The oracle's view of a model: f32 weights (a dict from ava_amd.synth) with their int8 copies
    made by orc_quantize_int8, as Model::set_int8 does (gpu/model.rs:949-991)."""

    def __init__(self, cfg: dict, params: dict):
        self.cfg = dict(cfg)
        self.params = params
        self._keep = []
        L = cfg["layers"]
        self.q8 = {}
        blocks = (_Block * L)()
        for i in range(L):
            bp = params["blocks"][i]
            blk = blocks[i]
            for name in _BLOCK_F32:
                if name in bp and bp[name] is not None:
                    setattr(blk, name, self._ptr(bp[name]))
            for name in _BLOCK_Q8:
                if name in bp and bp[name] is not None:
                    setattr(blk, name, self._qw(bp[name]))
        self.blocks = blocks
        head_w = np.ascontiguousarray(params["tok_emb"].T)
        self._keep.append(head_w)
        self.model = _Model(tok_emb=self._ptr(params["tok_emb"]),
                            head=self._qw(head_w),
                            final_norm=self._ptr(params["final_norm"]),
                            blocks=C.cast(blocks, C.POINTER(_Block)))
        c = self.cfg
        self.ccfg = _Cfg(vocab=c["vocab"], d=c["d"], layers=L, hidden=c["hidden"], kwta_k=c["kwta_k"],
                         heads=c["d"] // c["head_size"], head_size=c["head_size"], gate_rank=c["gate_rank"],
                         eng_block=c["eng_block"], eng_dim=c["eng_dim"], levels=c["levels"],
                         alif=int(c["alif"]), lif_scale=int(c["lif_scale"]),
                         value_residual=int(c["value_residual"]), dense=int(c["dense"]),
                         relu2=int(c["relu2"]), momentum=c["momentum"], cap=c["cap"],
                         eng_half=int(c.get("eng_half", 0) or 0), eng_heads=int(c.get("eng_heads", 1) or 1))
        self.head_q, self.head_s = self.q8[id(head_w)]
        # the cerebellum head (gpu/v51b.rs:18-32, 282-293): wiring from the fixed seed, the read-out W
        # (cbh.wo, zero at init: None), the online rate and half-life
        self.cb = int(c.get("cb_units", 0) or 0)
        if self.cb:
            from ava_amd import synth
            d = c["d"]
            self.cb_idx, self.cb_sgn = cb_wiring(2 * d, self.cb, synth.CB_FAN_IN, synth.CB_SEED)
            self.cb_k = self.cb // synth.CB_SPARSITY
            self.cb_w = params.get("cb_w")
            self.cb_lr = synth.cb_rate(params["tok_emb"], c["cb_eta"])
            self.cb_half = float(c.get("cb_half", 0.0) or 0.0)

    def _ptr(self, a):
        a = _c(a, np.float32)
        self._keep.append(a)
        return a.ctypes.data

    def _qw(self, w):
        q, s = quantize_int8(w)
        self._keep += [q, s]
        self.q8[id(w)] = (q, s)
        return _QW(q=q.ctypes.data, scale=s.ctypes.data, din=w.shape[0], dout=w.shape[1])

    def new_state(self, B, eng_cap=0, counts=False):
        """A zero state of B streams; counts: keep the least-read rule's per-slot reads and ages."""
        c = self.cfg
        L, d, hs = c["layers"], c["d"], c["head_size"]
        nh = d // hs
        de = c["eng_dim"]
        st = {
            "lif_v": np.zeros((L, B, d), np.float32), "lif_s": np.zeros((L, B, d), np.float32),
            "lif_a": np.zeros((L, B, d), np.float32),
            "mem_f": np.zeros((L, B, nh, hs, hs), np.float32), "mem_s": np.zeros((L, B, nh, hs, hs), np.float32),
            "eng_k": np.zeros((B, max(eng_cap, 1), de), np.float32),
            "eng_v": np.zeros((B, max(eng_cap, 1), de), np.float32),
            "eng_cap": eng_cap, "eng_len": 0,
        }
        if counts:
            st["eng_reads"] = np.zeros((B, max(eng_cap, 1)), np.float32)
            st["eng_age"] = np.zeros((B, max(eng_cap, 1)), np.float32)
        if self.cb:
            # the online table per stream (gpu/v51b.rs:340-367: delta, scale) and the last position's code
            st["cb_tab"] = np.zeros((B, self.cb, d), np.float32)
            st["cb_scale"] = np.ones(B, np.float64)
            st["cb_code"] = np.zeros((B, self.cb), np.float32)
        return st

    def forward(self, ids, state=None, planes=0, threads=1, trace=False, logits=True, force=None):
        """gpu/arch.rs:1407 forward_arch / gpu/state.rs:684 forward_with_state. ids [B, T].
        force: None, or {"spikes": int8 [L, B*T, d], "keep": bool/uint8 [L, B*T, H]} decisions that
        replace the oracle's own (its own are still traced: spikes, u, kth, and the LIF decision
        inputs vm, tht); forcing implies trace=True."""
        ids = _c(ids, np.int32)
        B, T = ids.shape
        c = self.cfg
        if state is None:
            state = self.new_state(B, eng_cap=T if c["eng_block"] >= 0 else 0)
        cst = _State(**{k: state[k].ctypes.data for k in ("lif_v", "lif_s", "lif_a", "mem_f", "mem_s",
                                                         "eng_k", "eng_v")},
                     eng_cap=state["eng_cap"], eng_len=state["eng_len"],
                     eng_reads=state["eng_reads"].ctypes.data if "eng_reads" in state else None,
                     eng_age=state["eng_age"].ctypes.data if "eng_age" in state else None)
        N = B * T
        cb = self.cb and logits
        out = np.empty((N, c["vocab"]), np.float32) if logits and not cb else None
        tr = None
        trd = {}
        if cb and not trace:
            trd = {"hf": np.empty((N, c["d"]), np.float32)}
            tr = _Trace(hf=trd["hf"].ctypes.data)
        if trace or force is not None:
            L, d, H = c["layers"], c["d"], c["hidden"]
            trd = {"spikes": np.empty((L, N, d), np.int8), "cur": np.empty((L, N, d), np.float32),
                   "u": np.empty((L, N, H), np.float32), "kth": np.empty((L, N), np.float32),
                   "memy": np.empty((L, N, d), np.float32), "x": np.empty((L, N, d), np.float32),
                   "hf": np.empty((N, d), np.float32), "vm": np.empty((L, N, d), np.float32),
                   "tht": np.empty((L, N, d), np.float32)}
            ptrs = {k: v.ctypes.data for k, v in trd.items()}
            if force is not None:
                fs = _c(force["spikes"], np.int8).reshape(L, N, d)
                fk = _c(force["keep"], np.uint8).reshape(L, N, H)
                trd["_force"] = (fs, fk)  # kept alive through the call
                ptrs.update(force_spikes=fs.ctypes.data, force_keep=fk.ctypes.data)
            tr = _Trace(**ptrs)
        rc = lib().orc_model_forward(C.byref(self.ccfg), C.byref(self.model), ids.ctypes.data, B, T,
                                     C.byref(cst), None if out is None else out.ctypes.data, planes, threads,
                                     None if tr is None else C.byref(tr))
        if rc != 0:
            raise RuntimeError(f"orc_model_forward failed ({rc})")
        state["eng_len"] = cst.eng_len
        if cb:
            # gpu/model/fstep/arch.rs:1045-1047: the final normed state, the cerebellum's correction, the head
            E = self.params["tok_emb"]
            hf = trd["hf"]
            xo = np.empty_like(hf)
            for n in range(N):
                bi = n // T
                code = cb_code(hf[n], E[ids.reshape(-1)[n]], self.cb_idx, self.cb_sgn, self.cb_k)
                xo[n] = cb_apply(hf[n], code, self.cb_w, state["cb_tab"][bi], float(state["cb_scale"][bi]))
                if n % T == T - 1:
                    state["cb_code"][bi] = code
            if planes <= 0:
                out = q8_matmul_ref(xo, self.head_q, self.head_s, threads)
            else:
                out = q8_matmul_planes(xo, planes, self.head_q, self.head_s, threads)
        return out, state, trd

    def cb_learn(self, logits, nxt, state):
        """gpu/fast4/cb.rs:25-84 per stream: logits [B, V] of each stream's last position, nxt [B]
        (a negative id: no step). Returns the nats per stream."""
        E = self.params["tok_emb"]
        nats = []
        for bi in range(len(nxt)):
            n, sc = cb_learn(logits[bi], int(nxt[bi]), E, state["cb_code"][bi], self.cb_lr, self.cb_half,
                             float(state["cb_scale"][bi]), state["cb_tab"][bi])
            state["cb_scale"][bi] = sc
            nats.append(n)
        return np.array(nats)
