"""The oracle's cerebellum head and online table (CPU), pinned against the reference's own properties.

gpu/v51b/tests.rs:321-387 (cerebellum_online_rule_is_the_gradient_and_learns):
  (a) one online step equals -lr times the gradient of that word's cross-entropy with respect to W,
  (b) the table's correction equals the same change folded into the read-out,
  (c) on a text read three times the loss of the later readings goes down;
plus an empty table adds nothing (ibid.), the wiring's stated form (gpu/v51b.rs:242-265), the code's
stated form (gpu/v51b.rs:327-337: the top G/32, relu, unit length) against a brute-force numpy
statement, and CB2's fading scale (gpu/v51b.rs:352-367, gpu/fast4/cb.rs:58-66).
"""
import numpy as np
import pytest

from ava_amd import synth
from oracle import oracle as O

SEED = synth.CB_SEED


def xorshift_wiring(inputs, g, fan_in, seed):
    """An independent statement of gpu/v51b.rs:242-265 with explicit 64-bit wrap."""
    m = (1 << 64) - 1
    s = (seed | 1) & m

    def nxt():
        nonlocal s
        s ^= (s << 13) & m
        s ^= s >> 7
        s ^= (s << 17) & m
        return s

    idx, sgn = [], []
    for _ in range(g):
        picked = []
        while len(picked) < min(fan_in, inputs):
            r = nxt() % inputs
            if r not in picked:
                picked.append(r)
        for r in picked:
            idx.append(r)
            sgn.append(0.5 if nxt() & 1 == 0 else -0.5)
    return np.array(idx, np.uint32).reshape(g, fan_in), np.array(sgn, np.float32).reshape(g, fan_in)


def test_cb_wiring_form():
    idx, sgn = O.cb_wiring(2 * 128, 512, 4, SEED)
    widx, wsgn = xorshift_wiring(256, 512, 4, SEED)
    assert np.array_equal(idx, widx) and np.array_equal(sgn, wsgn)
    assert idx.max() < 256 and all(len(set(r)) == 4 for r in idx.tolist())
    assert set(np.unique(sgn).tolist()) == {-0.5, 0.5}
    # both signs and every input are used at this size
    assert 0.4 < (sgn > 0).mean() < 0.6 and len(np.unique(idx)) == 256


def code_f64(xf, emb_row, idx, sgn, k):
    d = xf.shape[0]
    e = emb_row.astype(np.float64)
    u = np.concatenate([xf.astype(np.float64), e / np.sqrt(np.mean(e * e) + 1e-5)])
    h = (u[idx] * sgn).sum(1)
    kth = np.sort(h)[::-1][k - 1]
    a = np.where(h - kth >= 0, np.maximum(h, 0.0), 0.0)
    return a / (np.sqrt((a * a).sum()) + 1e-6), h


@pytest.mark.parametrize("d,g", [(128, 512), (64, 1024)])
def test_cb_code_is_top_k_relu_unit(d, g):
    rng = np.random.default_rng(d + g)
    idx, sgn = O.cb_wiring(2 * d, g, 4, SEED)
    k = g // 32
    for trial in range(4):
        xf = rng.standard_normal(d).astype(np.float32)
        emb = (rng.standard_normal(d) * 0.02).astype(np.float32)
        c = O.cb_code(xf, emb, idx, sgn, k)
        want, h = code_f64(xf, emb, idx, sgn, k)
        top = np.argsort(-h)[:k]
        assert (c != 0).sum() <= k and set(np.flatnonzero(c)) <= set(top.tolist())
        assert set(np.flatnonzero(c)) == set(top[h[top] > 0].tolist())
        assert np.max(np.abs(c - want)) < 1e-6
        assert abs(np.linalg.norm(c.astype(np.float64)) - 1.0) < 1e-5


def test_cb_apply_readout_and_table():
    rng = np.random.default_rng(3)
    d, g = 96, 256
    xf = rng.standard_normal(d).astype(np.float32)
    c = np.zeros(g, np.float32)
    on = rng.choice(g, 8, replace=False)
    c[on] = rng.random(8).astype(np.float32)
    w = rng.standard_normal((g, d)).astype(np.float32)
    tab = rng.standard_normal((g, d)).astype(np.float32)
    for scale in (1.0, 0.37):
        out = O.cb_apply(xf, c, w, tab, scale)
        want = xf.astype(np.float64) + c.astype(np.float64) @ w + scale * (c.astype(np.float64) @ tab)
        assert np.max(np.abs(out - want)) < 1e-5 * np.max(np.abs(want))
    # no read-out and no table: xf itself
    assert np.array_equal(O.cb_apply(xf, c), xf)


def test_cb_learn_step_is_minus_lr_gradient():
    """(a): logits = (xf + c.W) E^T; one step with the table at scale 1 equals -lr dCE/dW, the
    gradient taken by central differences on the winners' rows in float64."""
    rng = np.random.default_rng(5)
    d, g, V = 24, 64, 40
    E = (rng.standard_normal((V, d)) * 0.3).astype(np.float32)
    xf = rng.standard_normal(d).astype(np.float32)
    c = np.zeros(g, np.float32)
    on = np.sort(rng.choice(g, 5, replace=False))
    c[on] = rng.random(5).astype(np.float32)
    c /= np.linalg.norm(c)
    nxt, lr = 7, 0.5
    logits = (E.astype(np.float64) @ xf.astype(np.float64)).astype(np.float32)  # W = 0
    tab = np.zeros((g, d), np.float32)
    nats, sc = O.cb_learn(logits, nxt, E, c, lr, 0.0, 1.0, tab)
    assert sc == 1.0

    def ce(W):
        z = E.astype(np.float64) @ (xf + c.astype(np.float64) @ W)
        z = z - z.max()
        return -(z[nxt] - np.log(np.exp(z).sum()))

    assert abs(nats - ce(np.zeros((g, d)))) < 1e-5
    W0 = np.zeros((g, d))
    grad = np.zeros((g, d))
    h = 1e-4
    for u in on:
        for i in range(d):
            Wp, Wm = W0.copy(), W0.copy()
            Wp[u, i] += h
            Wm[u, i] -= h
            grad[u, i] = (ce(Wp) - ce(Wm)) / (2 * h)
    want = -lr * grad
    assert np.max(np.abs(tab - want)) < 1e-4 * max(np.max(np.abs(want)), 1.0)
    assert np.all(tab[np.setdiff1d(np.arange(g), on)] == 0)


def test_cb_learn_ignores_outside_vocab():
    logits = np.zeros(10, np.float32)
    tab = np.ones((4, 3), np.float32)
    c = np.array([1, 0, 0, 0], np.float32)
    nats, sc = O.cb_learn(logits, -1, np.ones((10, 3), np.float32), c, 0.1, 2.0, 1.0, tab)
    assert np.isnan(nats) and sc == 1.0 and np.all(tab == 1.0)


def test_cb_scale_fades_and_folds():
    """CB2: each step multiplies the scale by 2^(-1/half); below 1e-18 the table folds (scale back to
    1). The table as it acts (scale x delta) carries over the fold."""
    rng = np.random.default_rng(9)
    d, g, V, half = 8, 16, 12, 2.0
    E = rng.standard_normal((V, d)).astype(np.float32)
    c = np.zeros(g, np.float32)
    c[3] = 1.0
    tab = np.zeros((g, d), np.float32)
    sc = 1.0
    for t in range(1, 130):
        before = tab * sc
        nats, sc2 = O.cb_learn(rng.standard_normal(V).astype(np.float32), t % V, E, c, 0.1, half, sc, tab)
        fade = 2.0 ** (-1.0 / half)
        if sc * fade < 1e-18:
            assert sc2 == 1.0
        else:
            assert sc2 == sc * fade
        # untouched rows keep their effective value faded by exactly one step (fold: within f32 rounding)
        after = tab * sc2
        assert np.allclose(after[0], before[0] * fade, rtol=1e-6, atol=0)
        sc = sc2


def small_model(seed=0):
    cfg = synth.config("tiny_cb")
    params = synth.params(cfg, seed=seed)
    return cfg, params, O.OracleModel(cfg, params)


def test_cb_empty_table_adds_nothing():
    cfg, params, om = small_model()
    plain = dict(cfg, cb_units=0)
    op = O.OracleModel(plain, params)
    ids = np.random.default_rng(1).integers(0, cfg["vocab"], (2, 6)).astype(np.int32)
    a, _, _ = om.forward(ids, state=om.new_state(2, eng_cap=6))
    b, _, _ = op.forward(ids, state=op.new_state(2, eng_cap=6))
    assert np.array_equal(a, b)


def test_cb_table_equals_folded_readout():
    """(b): after learning on ten words, logits through the table equal logits with the table folded
    into the read-out W (scale x delta added to W, the table empty)."""
    cfg, params, om = small_model(2)
    toks = np.random.default_rng(4).integers(0, cfg["vocab"], 12).astype(np.int32)
    st = om.new_state(1, eng_cap=12)
    for j in range(10):
        lg, st, _ = om.forward(toks[None, j:j + 1], state=st)
        om.cb_learn(lg[-1:], [toks[j + 1]], st)
    assert np.any(st["cb_tab"] != 0)
    import copy
    st2 = copy.deepcopy(st)
    la, _, _ = om.forward(toks[None, 10:11], state=st)
    folded = dict(params, cb_w=(st2["cb_tab"][0].astype(np.float64) * st2["cb_scale"][0]).astype(np.float32))
    om2 = O.OracleModel(cfg, folded)
    st2["cb_tab"][:] = 0
    st2["cb_scale"][:] = 1.0
    lb, _, _ = om2.forward(toks[None, 10:11], state=st2)
    assert np.max(np.abs(la - lb)) < 1e-5 * max(1.0, np.max(np.abs(la)))


def test_cb_online_rule_learns_a_repeated_text():
    """(c): a 24-token text read three times in one stream, the rule on every word; the later reading's
    mean cross-entropy is lower."""
    cfg, params, om = small_model(6)
    toks = np.random.default_rng(8).integers(0, cfg["vocab"], 24).astype(np.int32)
    st = om.new_state(1, eng_cap=3 * 24)
    per = []
    for _ in range(3):
        tot = 0.0
        for j in range(23):
            lg, st, _ = om.forward(toks[None, j:j + 1], state=st)
            tot += om.cb_learn(lg[-1:], [toks[j + 1]], st)[0]
        per.append(tot / 23)
    assert per[2] < per[0] - 0.05, per
