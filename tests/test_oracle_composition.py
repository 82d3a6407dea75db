"""The oracle's block composition (orc_model_forward) pinned piece by piece against float64 numpy
statements of the reference's formulas, written from the reference (not from the oracle):

  - the embedding, the dense mix and the final norm + head (gpu/arch.rs:1407-1566, 1492-1500);
  - the spiking layer: cur = rms(x) . Win (1 - beta), the LIF scan with beta = sigmoid(beta_p),
    rho = sigmoid(arho), then x += s . Wout (gpu/arch.rs:1632-1695);
  - the memory: unit q, k, e = unit(k_raw + h We), the value residual, the per-channel gates
    log alpha = logsigmoid(h Wa + ba + off_c + h Wa1 Wa2), b = 2 sigmoid(h Wb + bb + h Wb1 Wb2), the
    recurrence of delta_rec with momentum and the bound (gpu/arch.rs:1091-1136, 1873-2020);
  - the read-out: head_norm(y) * silu(h Wg), then . Wo (gpu/model.rs:583-604);
  - the engram read: causal softmax attention per head, scale 1/sqrt(head size) (gpu/model.rs:543-562,
    gpu/memory.rs:610-700);
  - the sparse MLP: u = rms(x) . W1, kWTA (ties kept) with relu^2, then . W2 (gpu/arch.rs:1814-1855).

Each piece is isolated by zeroing the other paths' output weights (Wout, Wo, eWo, W2; the dense mix
weights where the stream should be plain), so the oracle's traced stream moves only by that piece.
The products are the reference's W8A32 (planes = 0) of the pinned quantizer. A swapped gate matrix,
a dropped offset, a wrong stream index or a transposed operand fails one of these. Also the scalar
helpers against closed forms at extreme arguments.
"""
import numpy as np
import pytest

from ava_amd import synth
from oracle import oracle as O

f64 = np.float64


# ----------------------------------------------------------------------------- float64 statements


def rms(x, g):
    """gpu/model.rs:458-462: x (mean(x^2) + 1e-5)^-1/2 gain."""
    x = x.astype(f64)
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + 1e-5) * np.asarray(g, f64)


def unit(x, hs):
    """gpu/model.rs:589-592 per head of hs: x (sum x^2 + 1e-6)^-1/2."""
    sh = x.shape
    x = x.reshape(sh[:-1] + (sh[-1] // hs, hs)).astype(f64)
    return (x / np.sqrt(np.sum(x * x, axis=-1, keepdims=True) + 1e-6)).reshape(sh)


def head_norm(y, hs):
    """gpu/model.rs:583-587: rms without gain per head."""
    sh = y.shape
    y = y.reshape(sh[:-1] + (sh[-1] // hs, hs)).astype(f64)
    return (y / np.sqrt(np.mean(y * y, axis=-1, keepdims=True) + 1e-5)).reshape(sh)


def sigmoid(z):
    return 1.0 / (1.0 + np.exp(-np.asarray(z, f64)))


def logsigmoid(z):
    return -np.logaddexp(0.0, -np.asarray(z, f64))


def mm(x, w):
    """int8::mm (gpu/int8.rs:672-683) in f64: x . dequant(quantize_int8(W))."""
    q, s = O.quantize_int8(w)
    return x.astype(f64) @ (q.astype(f64) * s.astype(f64)[None, :])


def kwta_relu2(u, k):
    """model::kwta_mask (gpu/model.rs:504-528, ties kept) with relu^2 (gpu/arch.rs:1820-1835)."""
    kth = -np.sort(-u, axis=1)[:, k - 1:k]
    a = np.maximum(u * (u - kth >= 0), 0.0)
    return a * a


def delta_rec(q, k, e, v, la, b, m, cap):
    """gpu/arch.rs:1091-1136 per (stream, head), f64: pred = e F; U = (b k) v^T - alpha (b e) pred;
    S = M S + U; F = clamp(alpha F + S); y = q F. Inputs [T, hs]."""
    hs = q.shape[1]
    F = np.zeros((hs, hs))
    S = np.zeros((hs, hs))
    y = np.zeros_like(q, dtype=f64)
    for t in range(q.shape[0]):
        al = np.exp(la[t])
        pred = e[t] @ F
        U = np.outer(b[t] * k[t], v[t]) - np.outer(al * b[t] * e[t], pred)
        S = m * S + U if m else U
        F = np.clip(al[:, None] * F + S, -cap, cap)
        y[t] = q[t] @ F
    return y, F, S


def attend(q, k, v, hd):
    """Causal softmax(q k^T / sqrt(hd)) v per head of hd over [T, de] rows."""
    T, de = q.shape
    out = np.zeros((T, de))
    for h in range(de // hd):
        sl = slice(h * hd, (h + 1) * hd)
        s = q[:, sl] @ k[:, sl].T / np.sqrt(hd)
        s = np.where(np.tril(np.ones((T, T), bool)), s, -np.inf)
        p = np.exp(s - s.max(axis=1, keepdims=True))
        out[:, sl] = (p / p.sum(axis=1, keepdims=True)) @ v[:, sl]
    return out


def relerr(a, b):
    return float(np.max(np.abs(np.asarray(a, f64) - b)) / max(np.max(np.abs(b)), 1e-30))


# ----------------------------------------------------------------------------- the setup


def setup(name="tiny", keep=(), dense_zero=False, seed=3, layers=3, B=2, T=20):
    """A model whose output paths not in `keep` (of wout, wo, ewo, w2) are zero; the oracle's traced
    W8A32 forward of seeded ids."""
    cfg = synth.config(name)
    cfg["layers"] = layers
    cfg["eng_block"] = 1
    prm = synth.params(cfg, seed=seed)
    rng = np.random.default_rng(seed + 100)
    for i, b in enumerate(prm["blocks"]):
        # gate weights large enough that each term moves the gates visibly
        b["wa"] = (rng.standard_normal(b["wa"].shape) * 0.2).astype(np.float32)
        b["wb"] = (rng.standard_normal(b["wb"].shape) * 0.2).astype(np.float32)
        b["wa1"] = (rng.standard_normal(b["wa1"].shape) * 0.2).astype(np.float32)
        b["wb1"] = (rng.standard_normal(b["wb1"].shape) * 0.2).astype(np.float32)
        b["we"] = (rng.standard_normal(b["we"].shape) * 0.1).astype(np.float32)
        for w in ("wout", "wo", "ewo", "w2"):
            if w in b and w not in keep:
                b[w] = np.zeros_like(b[w])
        if dense_zero:
            b["dense"] = np.zeros_like(b["dense"])
    ids = rng.integers(0, cfg["vocab"], (B, T)).astype(np.int32)
    om = O.OracleModel(cfg, prm)
    lo, so, tr = om.forward(ids, state=om.new_state(B, eng_cap=T), planes=0, threads=4, trace=True)
    return cfg, prm, ids, lo, so, tr


def block_inputs(prm, ids, tr, L):
    """The stream entering each block: the embedding, then the traced stream after each block."""
    x0 = prm["tok_emb"][ids.reshape(-1)].astype(f64)
    return [x0] + [tr["x"][i].astype(f64) for i in range(L - 1)]


# ----------------------------------------------------------------------------- scalar helpers


def test_sigmoid_and_log_sigmoid_closed_forms():
    """orc_sigmoid and orc_log_sigmoid (gpu/model.rs:465-467, 618-622) against 1/(1+e^-x) and
    -log(1+e^-x) in f64, including arguments where a naive form overflows or cancels."""
    xs = np.concatenate([np.linspace(-40, 40, 801), [-100.0, -88.0, -30.0, -1e-3, 0.0, 1e-3, 30.0, 88.0, 100.0]])
    for x in xs:
        s = float(O.sigmoid(x))
        want = float(sigmoid(np.float32(x)))
        assert abs(s - want) <= 4e-7 * max(want, 1e-30) + 1e-45, (x, s, want)
        ls = float(O.log_sigmoid(x))
        want = float(logsigmoid(np.float32(x)))
        assert np.isfinite(ls)
        assert abs(ls - want) <= 4e-7 * abs(want) + 1e-7, (x, ls, want)


def test_rmsnorm_closed_form():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((7, 96)) * np.array([1e-3, 1.0, 30.0, 1.0, 1.0, 1.0, 1e-8])[:, None]).astype(np.float32)
    g = rng.uniform(0.5, 2.0, 96).astype(np.float32)
    assert relerr(O.rmsnorm(x, g), rms(x, g)) < 1e-6


# ----------------------------------------------------------------------------- block pieces


def test_embedding_dense_mix_final_norm_and_head():
    """Every block's output path zeroed: each block's output is its input, and the stream moves only
    by the dense mix x_{i+1} = raw + sum_j w_j S_j (S_0 the embedding, S_{j+1} the raw output of block
    j); the logits are the head E^T of the final norm."""
    cfg, prm, ids, lo, so, tr = setup()
    L = cfg["layers"]
    x = prm["tok_emb"][ids.reshape(-1)].astype(f64)
    S = [x.copy()]
    for i in range(L):
        raw = x
        S.append(raw.copy())
        x = raw + sum(float(w) * s for w, s in zip(prm["blocks"][i]["dense"], S))
        assert relerr(tr["x"][i], x) < 1e-6, i
    want = mm(rms(x, prm["final_norm"]), np.ascontiguousarray(prm["tok_emb"].T))
    assert relerr(lo, want) < 1e-5


def test_dense_mix_one_hot_selects_its_stream():
    """Block 1's dense weights one-hot on stream j (block 0's zero, every path on): its output minus the
    same model's output with block 1's weights zero is exactly stream j: the embedding (j = 0), block 0's
    raw output (j = 1) or block 1's raw output (j = 2)."""
    cfg = synth.config("tiny")
    cfg["layers"] = 2
    prm = synth.params(cfg, seed=5)
    ids = np.random.default_rng(6).integers(0, cfg["vocab"], (1, 6)).astype(np.int32)

    def run(j):
        p2 = {**prm, "blocks": [dict(b) for b in prm["blocks"]]}
        for b in p2["blocks"]:
            b["dense"] = np.zeros_like(b["dense"])
        if j is not None:
            p2["blocks"][1]["dense"][j] = 1.0
        om = O.OracleModel(cfg, p2)
        return om.forward(ids, state=om.new_state(1, eng_cap=6), planes=0, trace=True)[2]["x"]

    base = run(None)
    streams = [prm["tok_emb"][ids.reshape(-1)], base[0], base[1]]  # S_0, S_1 = raw0, S_2 = raw1
    assert relerr(streams[1], streams[0]) > 1e-2 and relerr(streams[2], streams[1]) > 1e-2
    for j in range(3):
        x = run(j)
        assert np.array_equal(x[0], base[0])
        assert relerr(x[1].astype(f64) - base[1], streams[j].astype(f64)) < 1e-6, j


def test_spiking_layer_current_scan_and_wout():
    """Wout on, every other path off, no dense mix: cur = rms(x, lif_norm) . Win times (1 - beta),
    beta = sigmoid(beta_p); the spikes are the LIF scan of cur with (beta, theta, sigmoid(arho),
    again); the stream gains s . Wout."""
    cfg, prm, ids, lo, so, tr = setup(keep=("wout",), dense_zero=True)
    L, B, T, d = cfg["layers"], ids.shape[0], ids.shape[1], cfg["d"]
    xin = block_inputs(prm, ids, tr, L)
    for i in range(L):
        b = prm["blocks"][i]
        beta = sigmoid(b["beta_p"])
        cur = mm(rms(xin[i], b["lif_norm"]), b["win"]) * (1.0 - beta)[None, :]
        assert relerr(tr["cur"][i], cur) < 1e-5, i
        ps = np.concatenate([sigmoid(b["beta_p"]), b["theta"], sigmoid(b["arho"]), b["again"]]).astype(np.float32)
        spk, _, _, _ = O.lif_scan(tr["cur"][i].reshape(B, T, d), ps, levels=cfg["levels"], alif=cfg["alif"])
        assert np.array_equal(spk.reshape(B * T, d), tr["spikes"][i]), i
        assert 0.0 < np.mean(spk != 0) < 0.5
        assert relerr(tr["x"][i].astype(f64) - xin[i], mm(tr["spikes"][i].astype(f64), b["wout"])) < 1e-6, i


def memory_inputs(cfg, prm, i, h, v_first):
    """mem_arch (gpu/arch.rs:1873-1941), the per-channel branch, f64: q, k, e, v, log alpha, b [N, d]."""
    b = prm["blocks"][i]
    hs, d = cfg["head_size"], cfg["d"]
    nh = d // hs
    q = unit(mm(h, b["wq"]), hs)
    kraw = mm(h, b["wk"])
    k = unit(kraw, hs)
    v = mm(h, b["wv"])
    if cfg["value_residual"]:
        if i == 0:
            v_first[:] = [v]
        else:
            p0, p1 = float(b["vres"][0]), float(b["vres"][1])
            v = v * (1.0 + p0) + v_first[0] * p1
    za = h @ b["wa"].astype(f64) + b["ba"].astype(f64)  # f32 matmul in the reference: [N, nh]
    zb = h @ b["wb"].astype(f64) + b["bb"].astype(f64)
    za = np.repeat(za, hs, axis=1) + b["off"].astype(f64)[None, :] + (h @ b["wa1"].astype(f64)) @ b["wa2"].astype(f64)
    zb = np.repeat(zb, hs, axis=1) + (h @ b["wb1"].astype(f64)) @ b["wb2"].astype(f64)
    la = logsigmoid(za)
    bw = 2.0 * sigmoid(zb)
    e = unit(kraw + mm(h, b["we"]), hs)
    return q, k, e, v, la, bw


def test_memory_composition():
    """Every output path off: each block's memory reads h = rms(x_in, mem_norm) of the block's input.
    Its read-out (traced before the head norm) and its final F and S are the recurrence (delta_rec,
    f64) over the inputs mem_arch forms (per-channel gates with the offsets and the rank-32 read-outs,
    the erase key, the value residual of block 0's values)."""
    cfg, prm, ids, lo, so, tr = setup()
    L, B, T, d, hs = cfg["layers"], ids.shape[0], ids.shape[1], cfg["d"], cfg["head_size"]
    nh = d // hs
    xin = block_inputs(prm, ids, tr, L)
    v_first = [None]
    for i in range(L):
        h = rms(xin[i], prm["blocks"][i]["mem_norm"])
        q, k, e, v, la, bw = memory_inputs(cfg, prm, i, h, v_first)
        assert 0.3 < np.mean(bw) < 1.7 and np.std(la) > 0.05  # the gates vary
        y = np.zeros((B * T, d))
        for bi in range(B):
            rows = slice(bi * T, (bi + 1) * T)
            for hh in range(nh):
                c = slice(hh * hs, (hh + 1) * hs)
                yy, F, S = delta_rec(q[rows, c], k[rows, c], e[rows, c], v[rows, c], la[rows, c], bw[rows, c],
                                     cfg["momentum"], cfg["cap"])
                y[rows, c] = yy
                assert relerr(so["mem_f"][i, bi, hh], F) < 1e-5, (i, bi, hh)
                assert relerr(so["mem_s"][i, bi, hh], S) < 1e-5, (i, bi, hh)
        assert relerr(tr["memy"][i], y) < 1e-5, i


def test_memory_read_out_and_wo():
    """Wo on, every other path off, no dense mix: the stream gains (head_norm(y) * silu(h Wg)) . Wo
    with y the memory's traced read-out and h the memory's normed input."""
    cfg, prm, ids, lo, so, tr = setup(keep=("wo",), dense_zero=True)
    L, hs = cfg["layers"], cfg["head_size"]
    xin = block_inputs(prm, ids, tr, L)
    for i in range(L):
        b = prm["blocks"][i]
        h = rms(xin[i], b["mem_norm"])
        g = mm(h, b["wg"])
        out = mm(head_norm(tr["memy"][i], hs) * (g * sigmoid(g)), b["wo"])
        assert relerr(tr["x"][i].astype(f64) - xin[i], out) < 1e-5, i


@pytest.mark.parametrize("name", ["tiny", "tiny_heads"])
def test_engram_read_and_ewo(name):
    """eWo on, every other path off, no dense mix: the engram block's stream gains the causal softmax
    read of q, k, v = rms(x, eng_norm) . eWq, eWk, eWv per head (one head of 64, or heads of 32), . eWo."""
    cfg, prm, ids, lo, so, tr = setup(name=name, keep=("ewo",), dense_zero=True)
    L, B, T = cfg["layers"], ids.shape[0], ids.shape[1]
    xin = block_inputs(prm, ids, tr, L)
    i = cfg["eng_block"]
    b = prm["blocks"][i]
    h = rms(xin[i], b["eng_norm"])
    q, k, v = mm(h, b["ewq"]), mm(h, b["ewk"]), mm(h, b["ewv"])
    heads = max(1, int(cfg.get("eng_heads", 1) or 1))
    hd = cfg["eng_dim"] // heads
    o = np.concatenate([attend(q[r * T:(r + 1) * T], k[r * T:(r + 1) * T], v[r * T:(r + 1) * T], hd) for r in range(B)])
    assert relerr(tr["x"][i].astype(f64) - xin[i], mm(o, b["ewo"])) < 1e-5
    for j in range(L):
        if j != i:
            assert np.array_equal(tr["x"][j], xin[j].astype(np.float32)), j  # nothing else moves the stream


def test_sparse_mlp():
    """W2 on, every other path off, no dense mix: u = rms(x, mlp_norm) . W1; the stream gains
    kwta_relu2(u) . W2 (the k-th largest kept with ties, relu, squared)."""
    cfg, prm, ids, lo, so, tr = setup(keep=("w2",), dense_zero=True)
    L = cfg["layers"]
    xin = block_inputs(prm, ids, tr, L)
    for i in range(L):
        b = prm["blocks"][i]
        u = mm(rms(xin[i], b["mlp_norm"]), b["w1"])
        assert relerr(tr["u"][i], u) < 1e-5, i
        a = kwta_relu2(tr["u"][i].astype(f64), cfg["kwta_k"])
        assert relerr(tr["x"][i].astype(f64) - xin[i], mm(a, b["w2"])) < 1e-5, i


def test_value_residual_zero_is_the_identity():
    """vres = 0 leaves each block's values as they are (gpu/arch.rs:1903-1912, '(1 + p0) v + p1 v0:
    with p = 0 the values exactly'): the memory read-outs equal those of a model without the residual."""
    outs = []
    for vr in (True, False):
        cfg = synth.config("tiny")
        cfg["value_residual"] = vr
        prm = synth.params(cfg, seed=8)
        for b in prm["blocks"]:
            b["vres"] = np.zeros(2, np.float32)
        ids = np.random.default_rng(9).integers(0, cfg["vocab"], (2, 10)).astype(np.int32)
        om = O.OracleModel(cfg, prm)
        outs.append(om.forward(ids, state=om.new_state(2, eng_cap=10), planes=0, trace=True))
    assert np.array_equal(outs[0][0], outs[1][0])
    assert np.array_equal(outs[0][2]["memy"], outs[1][2]["memy"])


def test_large_gate_projection_makes_silu_the_identity():
    """silu(g) = g sigmoid(g) -> g for large g: with Wg scaled so h Wg is large and positive, the read-out
    path equals head_norm(y) * (h Wg) to rounding."""
    cfg, prm, ids, lo, so, tr = setup(keep=("wo",), dense_zero=True)
    L, hs = cfg["layers"], cfg["head_size"]
    prm2 = {**prm, "blocks": [dict(b) for b in prm["blocks"]]}
    rng = np.random.default_rng(11)
    for b in prm2["blocks"]:
        # a Wg with large entries, so many gate projections are far past the knee of silu
        b["wg"] = (rng.standard_normal((cfg["d"], cfg["d"])) * 4.0).astype(np.float32)
        b["mem_norm"] = np.abs(b["mem_norm"]).astype(np.float32)
    om = O.OracleModel(cfg, prm2)
    lo2, so2, tr2 = om.forward(ids, state=om.new_state(ids.shape[0], eng_cap=ids.shape[1]), planes=0, trace=True)
    xin = block_inputs(prm2, ids, tr2, L)
    i = 0
    h = rms(xin[i], prm2["blocks"][i]["mem_norm"])
    g = mm(h, prm2["blocks"][i]["wg"])
    big = g > 20.0
    assert np.mean(big) > 0.1
    gated = head_norm(tr2["memy"][i], hs) * (g * sigmoid(g))
    plain = head_norm(tr2["memy"][i], hs) * g
    assert np.max(np.abs(gated - plain)[big] / np.abs(plain[big])) < 1e-7


def test_every_path_on_reads_the_stream_after_the_previous_path():
    """Every output path on (no dense mix), one float64 statement of each whole block from its traced
    input: the memory reads rms(x_in + s . Wout), not the block input (gpu/arch.rs:1695-1705); the engram
    reads the stream after the memory's read-out was added; the MLP reads the stream after the engram's
    add; the block's output is the sum of all four. The other tests turn one path on at a time, so
    they do not fix which stream each later part reads."""
    cfg, prm, ids, lo, so, tr = setup(keep=("wout", "wo", "ewo", "w2"), dense_zero=True)
    L, B, T, d, hs = cfg["layers"], ids.shape[0], ids.shape[1], cfg["d"], cfg["head_size"]
    nh = d // hs
    xin = block_inputs(prm, ids, tr, L)
    v_first = [None]
    heads = max(1, int(cfg.get("eng_heads", 1) or 1))
    for i in range(L):
        b = prm["blocks"][i]
        x1 = xin[i] + mm(tr["spikes"][i].astype(f64), b["wout"])
        h = rms(x1, b["mem_norm"])
        # the spiking layer's add moves the memory's input visibly, so reading x_in would fail below
        assert relerr(rms(xin[i], b["mem_norm"]), h) > 1e-2
        q, k, e, v, la, bw = memory_inputs(cfg, prm, i, h, v_first)
        y = np.zeros((B * T, d))
        for bi in range(B):
            rows = slice(bi * T, (bi + 1) * T)
            for hh in range(nh):
                c = slice(hh * hs, (hh + 1) * hs)
                y[rows, c] = delta_rec(q[rows, c], k[rows, c], e[rows, c], v[rows, c], la[rows, c], bw[rows, c],
                                       cfg["momentum"], cfg["cap"])[0]
        assert relerr(tr["memy"][i], y) < 1e-4, i
        g = mm(h, b["wg"])
        x2 = x1 + mm(head_norm(tr["memy"][i], hs) * (g * sigmoid(g)), b["wo"])
        x3 = x2
        if i == cfg["eng_block"]:
            he = rms(x2, b["eng_norm"])
            assert relerr(rms(x1, b["eng_norm"]), he) > 1e-2
            eq, ek, ev = mm(he, b["ewq"]), mm(he, b["ewk"]), mm(he, b["ewv"])
            hd = cfg["eng_dim"] // heads
            o = np.concatenate([attend(eq[r * T:(r + 1) * T], ek[r * T:(r + 1) * T], ev[r * T:(r + 1) * T], hd)
                                for r in range(B)])
            x3 = x2 + mm(o, b["ewo"])
        hm = rms(x3, b["mlp_norm"])
        assert relerr(rms(x1 if i != cfg["eng_block"] else x2, b["mlp_norm"]), hm) > 1e-3
        u = mm(hm, b["w1"])
        assert relerr(tr["u"][i], u) < 1e-4, i
        x4 = x3 + mm(kwta_relu2(tr["u"][i].astype(f64), cfg["kwta_k"]), b["w2"])
        assert relerr(tr["x"][i], x4) < 1e-4, i
