"""The engram store's least-read eviction in the oracle (gpu/state.rs:518-590, gpu/memory.rs:700-738),
pinned by closed forms and by the reference's own test (gpu/state/tests.rs:238-285, engram_cap_rules).

With the engram's key projection zeroed every score is 0, so each query attends uniformly over the
slots it sees: query i of a first call of t tokens gives 1/(i + 1) to each slot j <= i, and slot j's
read mass (its own query left out) is H(t) - H(j + 1), with H the harmonic numbers; a second call of u
tokens adds sum_{i<u} 1/(n0 + i + 1) to every old slot. Ages: t - 1 - j after the first call, + u after
the second.
"""
import numpy as np

from ava_amd import synth
from oracle import oracle as O


def model(name="tiny", zero_keys=False, seed=7):
    cfg = synth.config(name)
    prm = synth.params(cfg, seed=seed)
    if zero_keys:
        blk = prm["blocks"][cfg["eng_block"]]
        blk["ewk"] = np.zeros_like(blk["ewk"])
    return cfg, prm


def harmonic(n):
    return float(np.sum(1.0 / np.arange(1, n + 1, dtype=np.float64))) if n > 0 else 0.0


def test_reads_and_ages_uniform_closed_form():
    for name in ("tiny", "tiny_heads"):
        cfg, prm = model(name, zero_keys=True)
        om = O.OracleModel(cfg, prm)
        t, u = 20, 7
        ids = np.random.default_rng(1).integers(0, cfg["vocab"], (2, t + u)).astype(np.int32)
        st = om.new_state(2, eng_cap=t + u, counts=True)
        om.forward(ids[:, :t], state=st, planes=3)
        want = np.array([harmonic(t) - harmonic(j + 1) for j in range(t)])
        for r in range(2):
            assert np.allclose(st["eng_reads"][r, :t], want, rtol=1e-5, atol=1e-6), name
            assert np.array_equal(st["eng_age"][r, :t], np.arange(t - 1, -1, -1, dtype=np.float32))
        om.forward(ids[:, t:], state=st, planes=3)
        add = sum(1.0 / (t + i + 1) for i in range(u))
        want2 = np.concatenate([want + add, [harmonic(t + u) - harmonic(t + j + 1) for j in range(u)]])
        for r in range(2):
            assert np.allclose(st["eng_reads"][r, :t + u], want2, rtol=1e-5, atol=1e-6), name
            assert np.array_equal(st["eng_age"][r, :t], np.arange(t - 1, -1, -1, dtype=np.float32) + u)
            assert np.array_equal(st["eng_age"][r, t:t + u], np.arange(u - 1, -1, -1, dtype=np.float32))


def test_reads_sum_to_the_mass_off_the_own_key():
    """Every query's softmax sums to one over the slots it sees, its own included: the counts of a
    first call add up to t minus the mass the queries gave their own keys (all below 1, so the total is
    below t and, with t queries of which the first sees only itself, above 0)."""
    cfg, prm = model("tiny_heads", seed=3)
    om = O.OracleModel(cfg, prm)
    t = 24
    ids = np.random.default_rng(4).integers(0, cfg["vocab"], (1, t)).astype(np.int32)
    st = om.new_state(1, eng_cap=t, counts=True)
    om.forward(ids, state=st, planes=3)
    tot = float(np.sum(st["eng_reads"][0, :t], dtype=np.float64))
    assert 0.0 < tot < t - 1 + 1e-4
    assert np.all(st["eng_reads"][0, :t] >= 0.0) and st["eng_reads"][0, t - 1] == 0.0


def test_engram_cap_rules_least_read():
    """gpu/state/tests.rs:259-277: the counted store of a first call (cap never reached) has age t1 - 1
    at slot 0 and 0 at the last; a least-read cap of 8 keeps the slots ranked last by (seen later, reads
    per later query, index), in store order; the oldest rule keeps the last 8."""
    cfg, prm = model("tiny", seed=12)
    om = O.OracleModel(cfg, prm)
    t1 = 20
    ids = np.random.default_rng(61).integers(0, cfg["vocab"], (1, t1)).astype(np.int32)
    counted = om.new_state(1, eng_cap=t1, counts=True)
    om.forward(ids, state=counted, planes=3)
    reads, age = counted["eng_reads"][0, :t1].copy(), counted["eng_age"][0, :t1].copy()
    assert age[0] == t1 - 1 and age[t1 - 1] == 0.0
    rank = sorted((1, float(reads[j] / age[j]), j) if age[j] >= 1.0 else (2, 0.0, j) for j in range(t1))
    keep = sorted(j for _, _, j in rank[t1 - 8:])
    lr = om.new_state(1, eng_cap=t1, counts=True)
    om.forward(ids, state=lr, planes=3)
    O.evict_engram(lr, 8, "least-read")
    assert lr["eng_len"] == 8
    assert np.array_equal(lr["eng_k"][0, :8], counted["eng_k"][0, keep])
    assert np.array_equal(lr["eng_reads"][0, :8], reads[keep]) and np.array_equal(lr["eng_age"][0, :8], age[keep])
    old = om.new_state(1, eng_cap=t1)
    om.forward(ids, state=old, planes=3)
    O.evict_engram(old, 8, "oldest")
    assert np.array_equal(old["eng_k"][0, :8], counted["eng_k"][0, t1 - 8:t1])
    # the least-read rule kept a different set than the oldest rule here (the test exercises the ranking)
    assert keep != list(range(t1 - 8, t1))
