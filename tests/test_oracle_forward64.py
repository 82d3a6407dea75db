"""oracle/forward64.py (the float64 reference point of the block stack's parity test) against the f32
oracle forward under the same forced decisions: on short sequences, where the stack's conditioning is
mild, the two agree to f32 rounding in every output and state. A planted mistake in the f32 oracle's
composition (one of the six the composition tests plant) would also separate them, so this fixes
forward64's composition to the pinned oracle's."""
import numpy as np
import pytest

from ava_amd import synth
from oracle import oracle as O
from oracle.forward64 import forward64


def rel(a, b):
    return float(np.max(np.abs(np.asarray(a, np.float64) - b)) / max(np.max(np.abs(b)), 1e-30))


@pytest.mark.parametrize("name,B,T", [("tiny", 2, 24), ("tiny_heads", 2, 17), ("small", 1, 40)])
def test_forward64_matches_the_f32_oracle_on_short_sequences(name, B, T):
    cfg = synth.config(name)
    prm = synth.params(cfg, seed=31)
    ids = np.random.default_rng(32).integers(0, cfg["vocab"], (B, T)).astype(np.int32)
    om = O.OracleModel(cfg, prm)
    _, _, tr = om.forward(ids, state=om.new_state(B, eng_cap=T), planes=0, threads=4, trace=True)
    keep = tr["u"] - tr["kth"][:, :, None] >= 0.0
    dec = {"spikes": tr["spikes"], "keep": keep.astype(np.uint8)}
    lo, so, _ = om.forward(ids, state=om.new_state(B, eng_cap=T), planes=0, threads=4, force=dec)
    l64, s64 = forward64(cfg, prm, ids, dec)
    assert rel(lo, l64) < 2e-5
    for k in ("lif_v", "lif_a", "mem_f", "mem_s"):
        for i in range(cfg["layers"]):
            assert rel(so[k][i], s64[k][i]) < 2e-5, (k, i, rel(so[k][i], s64[k][i]))
    assert np.array_equal(so["lif_s"], s64["lif_s"].astype(np.float32))
    # the memory grows state worth comparing, and the decisions vary
    assert np.max(np.abs(s64["mem_f"])) > 1e-2 and 0.0 < np.mean(tr["spikes"] != 0) < 0.5


def test_forward64_sees_a_changed_decision():
    """One flipped spike in block 0 changes the float64 forward's later state: the forced decisions are
    what it follows."""
    cfg = synth.config("tiny")
    prm = synth.params(cfg, seed=33)
    ids = np.random.default_rng(34).integers(0, cfg["vocab"], (1, 12)).astype(np.int32)
    om = O.OracleModel(cfg, prm)
    _, _, tr = om.forward(ids, state=om.new_state(1, eng_cap=12), planes=0, trace=True)
    dec = {"spikes": tr["spikes"].copy(), "keep": (tr["u"] - tr["kth"][:, :, None] >= 0.0).astype(np.uint8)}
    _, s1 = forward64(cfg, prm, ids, dec)
    dec["spikes"][0, 3, 5] = 2 - dec["spikes"][0, 3, 5]
    _, s2 = forward64(cfg, prm, ids, dec)
    assert rel(s2["mem_f"][1], s1["mem_f"][1]) > 1e-4


def test_float64_memory_against_numpy_rule_with_the_bound():
    """orc_mem_rec_f64d (forward64's memory) against a numpy statement of the bounded rule
    (gpu/arch.rs:1084-1136, mem_gen.rs:20-28: r = F^T e; U = (b k) v^T - (a b e) r^T; S = M S + U;
    F = clip(diag(a) F + S, +-cap); y = F^T q) with a cap that binds, and without momentum."""
    rng = np.random.default_rng(7)
    BH, T, hs = 3, 15, 16
    q, k, e, v = (rng.standard_normal((BH, T, hs)) for _ in range(4))
    al = rng.uniform(0.8, 1.0, (BH, T, hs))
    b = rng.uniform(0.2, 1.8, (BH, T, hs))
    for M, cap in ((0.5, 0.4), (0.0, np.inf)):
        y, F, S = O.mem_rec_f64d(q, k, e, v, al, b, m=M, cap=cap)
        hit = 0
        for n in range(BH):
            Fm, Sm = np.zeros((hs, hs)), np.zeros((hs, hs))
            for t in range(T):
                r = Fm.T @ e[n, t]
                U = np.outer(b[n, t] * k[n, t], v[n, t]) - np.outer(al[n, t] * b[n, t] * e[n, t], r)
                Sm = M * Sm + U if M else U
                raw = al[n, t][:, None] * Fm + Sm
                hit += int(np.sum(np.abs(raw) > cap))
                Fm = np.clip(raw, -cap, cap)
                # float64 in both, summed in different orders: agreement to ~1e-15 of the magnitudes
                sc = max(1.0, np.max(np.abs(Fm)))
                assert np.max(np.abs(y[n, t] - Fm.T @ q[n, t])) < 1e-12 * sc * hs
            assert np.max(np.abs(F[n] - Fm)) < 1e-12 * max(1.0, np.max(np.abs(Fm)))
            if M:
                assert np.max(np.abs(S[n] - Sm)) < 1e-12 * max(1.0, np.max(np.abs(Sm)))
        assert (hit > 0) == np.isfinite(cap)
