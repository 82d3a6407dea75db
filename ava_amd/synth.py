"""Configurations and seeded random-init weights of the Ava-0.4-shaped block stack.

The block recipe is Ava 0.4's (release/ava-0.4/arch.txt:1): int2 spikes with ALIF and a per-neuron
threshold, --lif-scale, per-channel memory gates with an erase key, momentum 0.5, the value
residual, kWTA 1/4 with relu2, the dense residual, head size 64; plus one single-head engram read
(d = 64) in block 4, as the benchmark configurations name it. The ten optional "brain parts" of
Ava 0.4 are not part of this path.

Weights follow the benchmark configurations: N(0, 0.02) for every projection (quantized to int8
per output column by the library), U(1.5, 4.5) leak logits, threshold 1, ALIF decay 0.95 and gain
0.05. Parameters the reference initialises at zero (the gate low-rank read-outs, the erase-key
projection, the value-residual and dense mixing weights) get small random values here so that
every term of the forward is exercised. All arrays are float32 numpy, keyed as the reference's
VarMap names them (gpu/arch.rs:806-860: b{i}.mem.*, b{i}.hebb.*).
"""
from __future__ import annotations

import numpy as np

GATE_RANK = 32  # gpu/arch.rs:80
MEM_CAP = 1e5  # gpu/mem_gen.rs:28
FIXED_TS = (5.0, 8.0)  # gpu/arch.rs:91


def config(name: str) -> dict:
    """Named configurations: "ava04_d512" (config[0]), "ava04_d1024" (config[3]), "ava04_d1024_decode"
    (config[4]), "ava04_d1024_heads" (config[3] with the engram's reference geometry: 32 heads of 32),
    "tiny", "small", "tiny_heads" and "tiny_cb" (tests). cb_units > 0 adds the cerebellum head
    (gpu/v51b.rs:18-32) with its online table: cb_eta sets the rate as cb_rate, cb_half the
    table's half-life in tokens (<= 0: it never fades)."""
    base = dict(levels=2, alif=True, lif_scale=True, value_residual=True, dense=True, relu2=True,
                momentum=0.5, cap=MEM_CAP, head_size=64, gate_rank=GATE_RANK, eng_dim=64)
    if name == "ava04_d512":
        base.update(vocab=8192, d=512, layers=8, hidden=2048, kwta_k=512, eng_block=4)
    elif name == "ava04_d1024":
        base.update(vocab=8192, d=1024, layers=8, hidden=4096, kwta_k=1024, eng_block=4)
    elif name == "tiny":
        base.update(vocab=256, d=128, layers=2, hidden=512, kwta_k=128, eng_block=1)
    elif name == "small":
        base.update(vocab=512, d=256, layers=3, hidden=1024, kwta_k=256, eng_block=1)
    elif name == "tiny_heads":
        # the engram at the reference's geometry: d / 32 heads of 32 over the whole width (gpu/memory.rs:610-700)
        base.update(vocab=256, d=128, layers=2, hidden=512, kwta_k=128, eng_block=1, eng_dim=128, eng_heads=4)
    elif name == "ava04_d1024_heads":
        # config[3]'s shapes with the engram at the reference's geometry: 32 heads of 32, f32 store
        base.update(vocab=8192, d=1024, layers=8, hidden=4096, kwta_k=1024, eng_block=4, eng_dim=1024, eng_heads=32)
    elif name == "tiny_cb":
        base.update(vocab=256, d=128, layers=2, hidden=512, kwta_k=128, eng_block=1)
        base.update(cb_units=512, cb_eta=0.5, cb_half=256.0)
    elif name == "ava04_d1024_decode":
        # config[4]: config[3]'s shapes with the cerebellum head's online table as Ava 0.4 talks with it
        # (gpu/bin/ava_live.rs:61-64: 12,288 granule units, rate 0.3 / mean |E_v|^2, half-life 256 tokens)
        base.update(vocab=8192, d=1024, layers=8, hidden=4096, kwta_k=1024, eng_block=4)
        base.update(cb_units=12288, cb_eta=0.3, cb_half=256.0)
        base.update(eng_half=True)  # config[4]: an fp16 KV cache
    else:
        raise ValueError(f"unknown config {name!r}")
    return base


def gate_gammas(nh: int) -> np.ndarray:
    """gpu/arch.rs:656-666 (Timescales::Fixed): gamma_h = 1 - 2^-(5 + 3 h / (nh - 1))."""
    f = np.arange(nh, dtype=np.float64) / max(nh - 1, 1)
    return 1.0 - 2.0 ** -(FIXED_TS[0] + (FIXED_TS[1] - FIXED_TS[0]) * f)


def logit(p):
    p = np.asarray(p, np.float64)
    return np.log(p / (1.0 - p))


def params(cfg: dict, seed: int = 0) -> dict:
    rng = np.random.default_rng(seed)
    d, H, L, V = cfg["d"], cfg["hidden"], cfg["layers"], cfg["vocab"]
    hs, r, de = cfg["head_size"], cfg["gate_rank"], cfg["eng_dim"]
    nh = d // hs

    def n(*shape, std=0.02):
        return (rng.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float32)

    def const(shape, v):
        return np.full(shape, v, np.float32)

    off = np.repeat(logit(gate_gammas(nh)), hs).astype(np.float32)
    # The spiking layer's norm gain sets its input drive: with N(0, 0.02) weights the current's spread
    # is 0.02 sqrt(d), and after the (1 - beta) scaling the membranes would never reach threshold 1.
    # A gain of 3.2 / (0.02 sqrt(d)) puts about one unit-step in ten above threshold.
    lif_gain = np.float32(3.2 / (0.02 * np.sqrt(d)))
    blocks = []
    for i in range(L):
        b = {
            "lif_norm": const(d, lif_gain),
            "win": n(d, d),
            "beta_p": rng.uniform(1.5, 4.5, d).astype(np.float32),
            "theta": const(d, 1.0),
            "arho": const(d, float(logit(0.95))),
            "again": const(d, 0.05),
            "wout": n(d, d),
            "mem_norm": const(d, 1.0),
            "wq": n(d, d), "wk": n(d, d), "wv": n(d, d), "we": n(d, d), "wg": n(d, d), "wo": n(d, d),
            "wa": n(d, nh), "ba": n(nh, std=0.1), "wb": n(d, nh), "bb": n(nh, std=0.1),
            "off": off,
            "wa1": n(d, r), "wa2": n(r, d, std=0.05), "wb1": n(d, r), "wb2": n(r, d, std=0.05),
            "vres": np.array([0.1, 0.2], np.float32) if i > 0 else np.zeros(2, np.float32),
            "mlp_norm": const(d, 1.0),
            "w1": n(d, H), "w2": n(H, d),
            "dense": n(i + 2, std=0.05),
        }
        if i == cfg["eng_block"]:
            b.update(eng_norm=const(d, 1.0), ewq=n(d, de), ewk=n(d, de), ewv=n(d, de), ewo=n(de, d))
        blocks.append(b)
    return {"tok_emb": n(V, d), "final_norm": const(d, 1.0), "blocks": blocks}


CB_FAN_IN = 4  # gpu/v51b.rs:46-48
CB_SPARSITY = 32
CB_SEED = 0x51B0CE7E


def cb_rate(tok_emb: np.ndarray, eta: float) -> float:
    """gpu/v51b.rs:606-611 (Model::cb_rate): eta / mean |E_v|^2 = eta * V / sum(E^2), the sum in f32."""
    e2 = np.float32(np.sum(np.asarray(tok_emb, np.float32) ** 2, dtype=np.float32))
    return float(np.float32(eta * tok_emb.shape[0] / float(e2)))
