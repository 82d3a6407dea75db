"""A float64 statement of the block-stack forward with every discrete decision forced.

TEST INFRASTRUCTURE ONLY (as the rest of oracle/): nothing in the product path imports it.

orc_model_forward (ava_oracle.c) restates the reference's f32 loops, so it shares the reference's
rounding. On a deep stack over thousands of tokens the fast-weight recurrences amplify f32 rounding
past the state bars (heads that grow towards the +-1e5 bound), and two correct f32 implementations that
sum in different orders both drift from the exact result by about the same amount. This module is
the exact-arithmetic reference point for that comparison: the same composition in float64, the
decisions (spikes, the kWTA index set) forced from a trace so that it follows the same trajectory.
Each piece follows the reference's formulas (the same lines orc_model_forward cites):

  - embedding, dense mix, final norm and head: gpu/arch.rs:1407-1566, 1492-1500;
  - spiking layer: cur = rms(x, lif_norm) . Win times (1 - beta), beta = sigmoid(beta_p); the LIF
    recurrence of gpu/lif_gen.rs:171-180 with the forced spikes driving reset and trace; x += s . Wout
    (gpu/arch.rs:1632-1695);
  - memory: q, k unit per head, e = unit(k_raw + h We), the value residual, per-channel gates
    log alpha = logsigmoid(h Wa + ba + off + h Wa1 Wa2), b = 2 sigmoid(h Wb + bb + h Wb1 Wb2), the
    bounded delta_rec with momentum (gpu/arch.rs:1091-1136, 1873-2020); read-out head_norm(y) silu(h Wg)
    . Wo (gpu/model.rs:583-604);
  - engram read: causal softmax per head, scale 1/sqrt(head size) (gpu/memory.rs:610-700);
  - sparse MLP: relu(u mask)^2 . W2 with the forced mask (gpu/arch.rs:1814-1855).

Products use the pinned quantizer's weights (orc_quantize_int8) dequantized exactly, q x scale, so the
int8 model is the same model; only the arithmetic is exact. From a fresh state (no carried state and
an empty engram store), without the cerebellum head.
"""
from __future__ import annotations

import numpy as np

from . import oracle as O

f64 = np.float64


def _rms(x, g, eps=1e-5):
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * np.asarray(g, f64)


def _unit(x, hs):
    sh = x.shape
    z = x.reshape(sh[:-1] + (sh[-1] // hs, hs))
    return (z / np.sqrt(np.sum(z * z, axis=-1, keepdims=True) + 1e-6)).reshape(sh)


def _head_norm(y, hs):
    sh = y.shape
    z = y.reshape(sh[:-1] + (sh[-1] // hs, hs))
    return (z / np.sqrt(np.mean(z * z, axis=-1, keepdims=True) + 1e-5)).reshape(sh)


def _sigmoid(z):
    return 1.0 / (1.0 + np.exp(-z))


def _logsigmoid(z):
    return -np.logaddexp(0.0, -z)


class _Deq:
    """Dequantized int8 weights, q x scale per output column (gpu/int8.rs:59-84), computed once."""

    def __init__(self):
        self.cache = {}

    def __call__(self, w):
        key = id(w)
        if key not in self.cache:
            q, s = O.quantize_int8(np.ascontiguousarray(w, np.float32))
            self.cache[key] = (w, q.astype(f64) * s.astype(f64)[None, :])
        return self.cache[key][1]


def forward64(cfg, prm, ids, force):
    """The forward of ids [B, T] from a fresh state with the decisions force = {"spikes": int8 [L, B*T, d],
    "keep": bool/uint8 [L, B*T, H]} (rows b-major). Returns (logits [B*T, V], state) in float64, the
    state keyed as OracleModel's: lif_v, lif_s, lif_a [L, B, d], mem_f, mem_s [L, B, nh, hs, hs]."""
    if cfg.get("cb_units", 0):
        raise ValueError("forward64: the cerebellum head is not stated here")
    ids = np.asarray(ids)
    B, T = ids.shape
    N = B * T
    L, d, H, hs = cfg["layers"], cfg["d"], cfg["hidden"], cfg["head_size"]
    nh = d // hs
    M, cap = float(cfg["momentum"]), float(cfg["cap"])
    W = _Deq()
    spikes_f = np.asarray(force["spikes"]).reshape(L, N, d).astype(f64)
    keep_f = np.asarray(force["keep"]).reshape(L, N, H).astype(bool)
    st = {k: np.zeros((L, B, d)) for k in ("lif_v", "lif_s", "lif_a")}
    st["mem_f"] = np.zeros((L, B, nh, hs, hs))
    st["mem_s"] = np.zeros((L, B, nh, hs, hs))

    x = prm["tok_emb"][ids.reshape(-1)].astype(f64)
    streams = [x.copy()] if cfg["dense"] else None
    vfirst = None
    for i in range(L):
        b = prm["blocks"][i]
        # ---- spiking layer
        beta = _sigmoid(b["beta_p"].astype(f64))
        cur = _rms(x, b["lif_norm"]) @ W(b["win"])
        if cfg["lif_scale"]:
            cur = cur * (1.0 - beta)[None, :]
        th0 = b["theta"].astype(f64)
        rho = _sigmoid(b["arho"].astype(f64)) if cfg["alif"] else np.zeros(d)
        gain = b["again"].astype(f64) if cfg["alif"] else np.zeros(d)
        v = np.zeros((B, d))
        s = np.zeros((B, d))
        a = np.zeros((B, d))
        thp = th0 + a * gain if cfg["alif"] else np.broadcast_to(th0, (B, d)).copy()
        cur3 = cur.reshape(B, T, d)
        sp3 = spikes_f[i].reshape(B, T, d)
        for t in range(T):
            tht = th0
            if cfg["alif"]:
                a = a * rho + np.abs(s) * (1.0 - rho)
                tht = th0 + a * gain
            v = (v * beta + cur3[:, t]) - s * thp
            s = sp3[:, t]
            thp = tht
        st["lif_v"][i], st["lif_s"][i], st["lif_a"][i] = v, s, a
        x = x + spikes_f[i] @ W(b["wout"])

        # ---- fast-weight memory
        h = _rms(x, b["mem_norm"])
        q = _unit(h @ W(b["wq"]), hs)
        kr = h @ W(b["wk"])
        k = _unit(kr, hs)
        vv = h @ W(b["wv"])
        if cfg["value_residual"]:
            if i == 0:
                vfirst = vv.copy()
            else:
                vv = vv * (1.0 + float(b["vres"][0])) + vfirst * float(b["vres"][1])
        e = _unit(kr + h @ W(b["we"]), hs)
        g = h @ W(b["wg"])
        za = h @ b["wa"].astype(f64) + b["ba"].astype(f64)
        zb = h @ b["wb"].astype(f64) + b["bb"].astype(f64)
        za = np.repeat(za, hs, axis=1) + b["off"].astype(f64)[None, :] + \
            (h @ b["wa1"].astype(f64)) @ b["wa2"].astype(f64)
        zb = np.repeat(zb, hs, axis=1) + (h @ b["wb1"].astype(f64)) @ b["wb2"].astype(f64)
        al = np.exp(_logsigmoid(za))
        bw = 2.0 * _sigmoid(zb)

        def heads(z):  # [N, d] -> [B*nh, T, hs]
            return z.reshape(B, T, nh, hs).transpose(0, 2, 1, 3).reshape(B * nh, T, hs)

        hq, hk, he, hv, ha, hb = (heads(z) for z in (q, k, e, vv, al, bw))
        y, F, S = O.mem_rec_f64d(hq, hk, he, hv, ha, hb, m=M, cap=cap)
        st["mem_f"][i] = F.reshape(B, nh, hs, hs)
        st["mem_s"][i] = (S if M else np.zeros_like(S)).reshape(B, nh, hs, hs)
        y = y.reshape(B, nh, T, hs).transpose(0, 2, 1, 3).reshape(N, d)
        x = x + (_head_norm(y, hs) * (g * _sigmoid(g))) @ W(b["wo"])

        # ---- engram read
        if i == cfg["eng_block"]:
            he_ = _rms(x, b["eng_norm"])
            eq, ek, ev = he_ @ W(b["ewq"]), he_ @ W(b["ewk"]), he_ @ W(b["ewv"])
            if cfg.get("eng_half"):
                # the store holds binary16 keys and values (config[4]'s KV cache format)
                ek = ek.astype(np.float32).astype(np.float16).astype(f64)
                ev = ev.astype(np.float32).astype(np.float16).astype(f64)
            de = cfg["eng_dim"]
            enh = max(1, int(cfg.get("eng_heads", 1) or 1))
            hd = de // enh
            o = np.zeros((N, de))
            causal = np.tril(np.ones((T, T), bool))
            for r in range(B):
                rows = slice(r * T, (r + 1) * T)
                for hh in range(enh):
                    c = slice(hh * hd, (hh + 1) * hd)
                    sc = eq[rows, c] @ ek[rows, c].T / np.sqrt(hd)
                    sc = np.where(causal, sc, -np.inf)
                    p = np.exp(sc - sc.max(axis=1, keepdims=True))
                    o[rows, c] = (p / p.sum(axis=1, keepdims=True)) @ ev[rows, c]
            x = x + o @ W(b["ewo"])

        # ---- sparse MLP with the forced index set
        u = _rms(x, b["mlp_norm"]) @ W(b["w1"])
        act = np.maximum(u * keep_f[i], 0.0)
        if cfg["relu2"]:
            act = act * act
        x = x + act @ W(b["w2"])

        # ---- dense residual
        if cfg["dense"]:
            streams.append(x.copy())
            x = x + sum(float(w) * sj for w, sj in zip(b["dense"], streams))

    logits = _rms(x, prm["final_norm"]) @ W(np.ascontiguousarray(prm["tok_emb"].T))
    return logits, st
