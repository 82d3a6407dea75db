"""The reference's ops on the HIP path, with the reference's names and argument meaning.

Tensors are torch tensors on the GPU (torch is used for device memory and streams only); every
op calls libava_amd.so through the C ABI of include/ava.h and raises AvaError on a non-zero
status (the reference bail!s on shape, dtype and contiguity errors).

    QW.from_tensor(w)            int8.rs:76-79   (QW::from_tensor; W [din, dout], x·W)
    mm(x, qw, planes=3)          int8.rs:672-683 (int8::mm)
    mm_spikes(s, qw)             int8.rs:672-683 on integer inputs (exact)
    lif_gen(cur, beta, ...)      lif_gen.rs:86-130
    kwta_relu(u, k, relu2)       model.rs:504-528 + arch.rs:1820-1835
    mem_gen(q, k, e, v, la, b, m)   mem_gen.rs:127-137
    mem_chunk(q, k, e, v, la, b, m) delta_chunk / chunk_core (arch.rs:1151-1164, 1243-1327)
    delta_rule_from(q, k, v, beta, la, f0)   model.rs:744-799 (chunked, per-head gates)
    attend(q, ks, vs, n0)        model/fstep.rs:303-329 (one head of 64, causal, over a store)

The backward of the scans (the training step's kernels, gpu/lif.cu):
    lif_gen_bwd(cur, ps, g_spk, ...)      lifg_bwd_* (lif.cu:3222-3290) / lif_ref's gradient (arch.rs:964-1071)
    kwta_relu2_bwd(u, kth, ga)            relu2_bwd (lif.cu:4666-4679)
    mem_gen_bwd(q, k, e, v, la, b, dy, m) memg_bwd* (lif.cu:3411-3888) / delta_rec's gradient (arch.rs:1091-1136)
    dense_back(S, G, wf, base, ...)       dense_back (lif.cu:4922-4971)
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import torch

from ._lib import QW as _QWC, check, lib


def _stream():
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def _p(t):
    return C.c_void_p(t.data_ptr()) if t is not None else None


def _need(t, dtype, name):
    if not t.is_cuda:
        raise ValueError(f"{name}: a GPU tensor is required")
    if t.dtype != dtype:
        raise ValueError(f"{name}: dtype {t.dtype}, expected {dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name}: a contiguous tensor is required")


def ldk(k: int) -> int:
    return lib().ava_q8_ldk(k)


class QW:
    """One int8 weight matrix on the GPU: qt [dout][ldk] int8, scale [dout] f32."""

    def __init__(self, din, dout, qt, scale):
        self.din, self.dout, self.qt, self.scale = din, dout, qt, scale
        self.ldk = qt.shape[1]
        self.c = _QWC(din=din, dout=dout, ldk=self.ldk, qt=qt.data_ptr(), scale=scale.data_ptr())

    @staticmethod
    def from_tensor(w: torch.Tensor) -> "QW":
        _need(w, torch.float32, "QW.from_tensor")
        din, dout = w.shape
        qt = torch.empty((dout, ldk(din)), dtype=torch.int8, device=w.device)
        scale = torch.empty(dout, dtype=torch.float32, device=w.device)
        check(lib().ava_q8_pack(_p(w), din, dout, _p(qt), _p(scale), _stream()), "ava_q8_pack")
        return QW(din, dout, qt, scale)


def quant_rows(x: torch.Tensor, planes: int = 3):
    _need(x, torch.float32, "quant_rows")
    m, k = x.shape
    xq = torch.empty((planes, m, ldk(k)), dtype=torch.int8, device=x.device)
    xe = torch.empty(m, dtype=torch.int32, device=x.device)
    check(lib().ava_q8_quant_rows(_p(x), m, k, planes, _p(xq), _p(xe), _stream()), "ava_q8_quant_rows")
    return xq, xe


def gemm_acc(xq: torch.Tensor, w: QW):
    _need(xq, torch.int8, "gemm_acc")
    planes, m, _ = xq.shape
    acc = torch.empty((planes, m, w.dout), dtype=torch.int32, device=xq.device)
    check(lib().ava_q8_gemm_acc(_p(xq), planes, m, C.byref(w.c), _p(acc), _stream()), "ava_q8_gemm_acc")
    return acc


def mm(x: torch.Tensor, w: QW, planes: int = 3) -> torch.Tensor:
    _need(x, torch.float32, "mm")
    m, k = x.shape
    if k != w.din:
        raise ValueError(f"mm: input width {k}, the weights take {w.din}")
    y = torch.empty((m, w.dout), dtype=torch.float32, device=x.device)
    nbytes = lib().ava_q8_workspace(m, k, planes)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
    check(lib().ava_q8_matmul(_p(x), m, C.byref(w.c), planes, _p(y), _p(ws), nbytes, _stream()), "ava_q8_matmul")
    return y


def mm_spikes(s: torch.Tensor, w: QW) -> torch.Tensor:
    """s [m][din] int8 (din == ldk) or [m][ldk]."""
    _need(s, torch.int8, "mm_spikes")
    m, k = s.shape
    if k != w.ldk:
        raise ValueError(f"mm_spikes: input width {k}, expected ldk {w.ldk}")
    y = torch.empty((m, w.dout), dtype=torch.float32, device=s.device)
    check(lib().ava_q8_matmul_i8(_p(s), m, C.byref(w.c), _p(y), _stream()), "ava_q8_matmul_i8")
    return y


@dataclass
class LifState:
    """arch.rs:945-950: membrane v, last spikes s, ALIF trace a, each [B, d]."""
    v: torch.Tensor
    s: torch.Tensor
    a: torch.Tensor


def lif_gen(cur, beta, theta=None, alif=None, levels=2, signed=True, init=None, th_out=False):
    """lif_gen.rs:86-130: the LIF scan of cur [B, T, d]. Returns (spikes int8 [B, T, d], LifState[, th_T])."""
    _need(cur, torch.float32, "lif_gen")
    B, T, D = cur.shape
    dev = cur.device
    theta = torch.ones(D, dtype=torch.float32, device=dev) if theta is None else theta
    if alif is None:
        rho = torch.zeros(D, dtype=torch.float32, device=dev)
        gain = torch.zeros(D, dtype=torch.float32, device=dev)
    else:
        rho, gain = alif
    ps = torch.cat([beta, theta, rho, gain]).to(torch.float32).contiguous()
    if init is None:
        v = torch.zeros((B, D), dtype=torch.float32, device=dev)
        s = torch.zeros((B, D), dtype=torch.float32, device=dev)
        a = torch.zeros((B, D), dtype=torch.float32, device=dev)
    else:
        v, s, a = init.v.clone(), init.s.clone(), init.a.clone()
    spikes = torch.empty((B, T, D), dtype=torch.int8, device=dev)
    tho = torch.empty((B, D), dtype=torch.float32, device=dev) if th_out else None
    rc = lib().ava_lif_scan(_p(cur), B, T, D, _p(ps), _p(v), _p(s), _p(a), levels, int(signed),
                            int(alif is not None), _p(spikes), _p(tho), _stream())
    check(rc, "ava_lif_scan")
    st = LifState(v, s, a)
    return (spikes, st, tho) if th_out else (spikes, st)


def kwta_relu(u: torch.Tensor, k: int, relu2: bool = True):
    """relu(u · kwta_mask(u, k)), squared with relu2. Returns (a, kth)."""
    _need(u, torch.float32, "kwta_relu")
    n, h = u.shape
    a = torch.empty_like(u)
    kth = torch.empty(n, dtype=torch.float32, device=u.device)
    check(lib().ava_kwta(_p(u), n, h, k, int(relu2), _p(a), _p(kth), _stream()), "ava_kwta")
    return a, kth


def mem_gen(q, k, e, v, la, b, m=0.0, cap=1e5, F=None, S=None):
    """mem_gen.rs:127-137 with carried state: q, k, e, v [BH, T, hs]; la, b [BH, T, g].
    Returns (y, F, S)."""
    for t, nm in ((q, "q"), (k, "k"), (e, "e"), (v, "v"), (la, "la"), (b, "b")):
        _need(t, torch.float32, f"mem_gen {nm}")
    BH, T, hs = q.shape
    g = la.shape[2]
    F = torch.zeros((BH, hs, hs), dtype=torch.float32, device=q.device) if F is None else F.clone()
    S = torch.zeros((BH, hs, hs), dtype=torch.float32, device=q.device) if S is None else S.clone()
    y = torch.empty_like(q)
    check(lib().ava_mem_scan(_p(q), _p(k), _p(e), _p(v), _p(la), _p(b), BH, T, hs, g, float(m), float(cap),
                             _p(F), _p(S), _p(y), _stream()), "ava_mem_scan")
    return y, F, S


def mem_chunk(q, k, e, v, la, b, m=0.0, cap=1e5, F=None, S=None):
    """delta_chunk / chunk_core (arch.rs:1151-1164, 1243-1327): mem_gen's rule in chunks of 16 tokens,
    the bound on F applied at chunk ends. Same arguments and result as mem_gen. Returns (y, F, S)."""
    for t, nm in ((q, "q"), (k, "k"), (e, "e"), (v, "v"), (la, "la"), (b, "b")):
        _need(t, torch.float32, f"mem_chunk {nm}")
    BH, T, hs = q.shape
    g = la.shape[2]
    F = torch.zeros((BH, hs, hs), dtype=torch.float32, device=q.device) if F is None else F.clone()
    S = torch.zeros((BH, hs, hs), dtype=torch.float32, device=q.device) if S is None else S.clone()
    y = torch.empty_like(q)
    check(lib().ava_mem_chunk(_p(q), _p(k), _p(e), _p(v), _p(la), _p(b), BH, T, hs, g, float(m), float(cap),
                              _p(F), _p(S), _p(y), _stream()), "ava_mem_chunk")
    return y, F, S


def delta_rule_from(q, k, v, beta, la=None, f0=None, workspace=True):
    """model.rs:744-799 (per-head gates): q, k, v [BH, T, 64], beta and la (log alpha, None: alpha = 1)
    [BH, T]. Without gates and with workspace, the chunks' inverses are formed first for all chunks (the
    two-phase form, a workspace of BH x T x 64 floats); else one kernel walks the chunks. Returns (y, F)."""
    for t, nm in ((q, "q"), (k, "k"), (v, "v"), (beta, "beta")) + (((la, "la"),) if la is not None else ()):
        _need(t, torch.float32, f"delta_rule {nm}")
    BH, T, hs = q.shape
    F = torch.zeros((BH, hs, hs), dtype=torch.float32, device=q.device) if f0 is None else f0.clone()
    y = torch.empty_like(q)
    nb = lib().ava_delta_chunk_workspace(BH, T) if (la is None and workspace) else 0
    work = torch.empty(nb, dtype=torch.uint8, device=q.device) if nb else None
    check(lib().ava_delta_chunk(_p(q), _p(k), _p(v), _p(la), _p(beta), BH, T, hs, _p(F), _p(y), _p(work), nb,
                                _stream()), "ava_delta_chunk")
    return y, F


def lif_gen_bwd(cur, ps, g_spk, init=None, g_vT=None, g_aT=None, levels=2, signed=True, alif=True, slope=1.0,
                reset_grad=False, segments=False):
    """The LIF scan's backward from the initial state init (LifState; None: zeros), ps = beta | theta |
    rho | gain [4D]. Returns dict dI [B, T, D], dv0, da0, dbeta, drho, dgain [B, D] (the parameter
    gradients per stream: sum over dim 0). segments=True: ava_lif_scan_bwd_segments (parallel segments
    for few chains; the same values up to the association of the sums)."""
    _need(cur, torch.float32, "lif_gen_bwd cur")
    _need(g_spk, torch.float32, "lif_gen_bwd g_spk")
    _need(ps, torch.float32, "lif_gen_bwd ps")
    B, T, D = cur.shape
    dev = cur.device
    z = torch.zeros((B, D), dtype=torch.float32, device=dev)
    v0, s0, a0 = (z, z, z) if init is None else (init.v, init.s, init.a)
    for t, nm in ((v0, "v0"), (s0, "s0"), (a0, "a0"), (g_vT, "g_vT"), (g_aT, "g_aT")):
        if t is not None:
            _need(t, torch.float32, f"lif_gen_bwd {nm}")
    out = {n: torch.empty((B, D), dtype=torch.float32, device=dev) for n in ("dv0", "da0", "dbeta", "drho", "dgain")}
    out["dI"] = torch.empty_like(cur)
    if segments:
        nb = lib().ava_lif_scan_bwd_segments_workspace(B, T, D)
        ws = torch.empty(nb // 4, dtype=torch.float32, device=dev)
        check(lib().ava_lif_scan_bwd_segments(_p(cur), B, T, D, _p(ps), _p(v0), _p(s0), _p(a0), levels, int(signed),
                                              int(alif), float(slope), int(reset_grad), _p(g_spk), _p(g_vT),
                                              _p(g_aT), _p(out["dI"]), _p(out["dv0"]), _p(out["da0"]),
                                              _p(out["dbeta"]), _p(out["drho"]), _p(out["dgain"]), _p(ws), nb,
                                              _stream()), "ava_lif_scan_bwd_segments")
        return out
    check(lib().ava_lif_scan_bwd(_p(cur), B, T, D, _p(ps), _p(v0), _p(s0), _p(a0), levels, int(signed), int(alif),
                                 float(slope), int(reset_grad), _p(g_spk), _p(g_vT), _p(g_aT), _p(out["dI"]),
                                 _p(out["dv0"]), _p(out["da0"]), _p(out["dbeta"]), _p(out["drho"]),
                                 _p(out["dgain"]), _stream()), "ava_lif_scan_bwd")
    return out


def kwta_relu2_bwd(u, kth, ga):
    """gu = (u ga) 2 on the units kwta_relu kept (u - kth >= 0) with u > 0, else 0."""
    _need(u, torch.float32, "kwta_relu2_bwd u")
    _need(ga, torch.float32, "kwta_relu2_bwd ga")
    _need(kth, torch.float32, "kwta_relu2_bwd kth")
    n, h = u.shape
    gu = torch.empty_like(u)
    check(lib().ava_kwta_relu2_bwd(_p(u), _p(kth), n, h, _p(ga), _p(gu), _stream()), "ava_kwta_relu2_bwd")
    return gu


def mem_gen_bwd(q, k, e, v, la, b, dy, m=0.0, cap=1e5, F0=None, S0=None, dF_T=None, dS_T=None):
    """The backward of mem_gen from the initial state (F0, S0; None: zeros) with dL/dy = dy and the
    final state's gradients (None: zeros). Returns dict dq, dk, de, dv, dla, db, dF0, dS0."""
    for t, nm in ((q, "q"), (k, "k"), (e, "e"), (v, "v"), (la, "la"), (b, "b"), (dy, "dy"), (F0, "F0"), (S0, "S0"),
                  (dF_T, "dF_T"), (dS_T, "dS_T")):
        if t is not None:
            _need(t, torch.float32, f"mem_gen_bwd {nm}")
    BH, T, hs = q.shape
    g = la.shape[2]
    o = {n: torch.empty_like(q) for n in ("dq", "dk", "de", "dv")}
    o.update({n: torch.empty_like(la) for n in ("dla", "db")})
    o["dF0"] = torch.empty((BH, hs, hs), dtype=torch.float32, device=q.device)
    o["dS0"] = torch.zeros((BH, hs, hs), dtype=torch.float32, device=q.device)
    nbytes = lib().ava_mem_scan_bwd_workspace(BH, T, int(m != 0.0))
    work = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=q.device)
    check(lib().ava_mem_scan_bwd(_p(q), _p(k), _p(e), _p(v), _p(la), _p(b), BH, T, hs, g, float(m), float(cap),
                                 _p(F0), _p(S0), _p(dy), _p(dF_T), _p(dS_T), _p(o["dq"]), _p(o["dk"]), _p(o["de"]),
                                 _p(o["dv"]), _p(o["dla"]), _p(o["db"]), _p(o["dF0"]), _p(o["dS0"]), _p(work),
                                 nbytes, _stream()), "ava_mem_scan_bwd")
    return o


def dense_back(S, G, wf, base, col, i0, L, nd):
    """The dense mix's backward: S [R, M] streams, G [L, M] = dL/d(mix after block k), wf packed weights.
    Returns (out [M], dw [nd])."""
    for t, nm in ((S, "S"), (G, "G"), (wf, "wf"), (base, "base")):
        _need(t, torch.float32, f"dense_back {nm}")
    M = base.numel()
    out = torch.empty_like(base)
    dw = torch.empty(max(nd, 1), dtype=torch.float32, device=base.device)
    nf = lib().ava_dense_back_part_floats(M, nd)
    part = torch.empty(max(nf, 1), dtype=torch.float32, device=base.device)
    check(lib().ava_dense_back(_p(S), _p(G), _p(wf), _p(base), _p(out), _p(dw), col, i0, L, nd, M, _p(part), nf,
                               _stream()), "ava_dense_back")
    return out, dw[:nd]


def attend(q: torch.Tensor, ks: torch.Tensor, vs: torch.Tensor, n0: int, heads: int = 1) -> torch.Tensor:
    """model/fstep.rs:303-329 per stream and query: q [B, T, de]; ks, vs [B, cap, de] (float32 or
    float16) holding entries 0..n0+T-1; query t reads entries 0..n0+t. heads = 1: one head of 64;
    heads > 1: heads of de / heads (32 or 64) side by side in each row, as memory::read
    (gpu/memory.rs:610-700). Returns out [B, T, de]."""
    _need(q, torch.float32, "attend q")
    for t, nm in ((ks, "ks"), (vs, "vs")):
        _need(t, ks.dtype, f"attend {nm}")
    if ks.dtype not in (torch.float32, torch.float16):
        raise ValueError("attend: the store is float32 or float16")
    B, T, de = q.shape
    cap = ks.shape[1]
    if ks.shape != vs.shape or ks.shape[0] != B or ks.shape[2] != de:
        raise ValueError("attend: q [B, T, de], ks and vs [B, cap, de] are required")
    out = torch.empty_like(q)
    half = int(ks.dtype == torch.float16)
    if heads == 1:
        if de != 64:
            raise ValueError("attend: one head of 64 dims (heads > 1 for wider rows)")
        n = lib().ava_attend_part_floats(B, T, n0)
        part = torch.empty(max(n, 1), dtype=torch.float32, device=q.device)
        check(lib().ava_attend(_p(q), 64, _p(ks), _p(vs), half, cap, n0, B, T, _p(out), _p(part), n, _stream()),
              "ava_attend")
        return out
    n = lib().ava_attend_heads_part_floats(B, T, n0, de, heads)
    part = torch.empty(max(n, 1), dtype=torch.float32, device=q.device)
    check(lib().ava_attend_heads(_p(q), de, _p(ks), _p(vs), half, cap, n0, B, T, de, heads, _p(out), _p(part), n,
                                 _stream()), "ava_attend_heads")
    return out
