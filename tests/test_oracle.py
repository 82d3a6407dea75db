"""The CPU oracle pinned against the reference's own known answers and against independent checks.

Each test names the reference test or property it restates (paths relative to the reference's
design-tests/nn/). A plausible slip in the oracle (a wrong sign, a dropped term, an index or
rounding mistake) fails at least one of them: the hand-worked spike trains, the straight-through
restatement of lif_ref, brute-force sorts, float64 products and recurrences, and closed-form
invariants of the delta rule.
"""
import numpy as np
import pytest

from oracle import oracle as O

F = np.float32


def unit_noise(n, seed):
    """gpu/testkit.rs:24-35: xorshift, uniform on +-sqrt(3)."""
    mask = (1 << 64) - 1
    x = ((seed * 0x9E3779B97F4A7C15) & mask) | 1
    out = np.empty(n, np.float32)
    for i in range(n):
        x ^= (x << 13) & mask
        x ^= x >> 7
        x ^= (x << 17) & mask
        u = (x >> 11) / float(1 << 53)
        out[i] = np.float32((u * 2.0 - 1.0) * np.sqrt(3.0))
    return out


def ps_of(beta, theta=None, rho=None, gain=None):
    d = len(beta)
    z = np.zeros(d, F)
    return np.concatenate([beta, np.ones(d, F) if theta is None else theta,
                           z if rho is None else rho, z if gain is None else gain]).astype(F)


# ----------------------------------------------------------------------------- LIF


def test_lif_integer_spikes_by_hand():
    """gpu/arch/tests.rs:433-445 (beta 0, theta 1)."""
    cur = np.array([2.5, -1.2, 0.3, -3.0, 1.0, 0.99], F).reshape(1, 6, 1)
    ps = ps_of(np.zeros(1, F))
    for levels, signed, want in [(1, True, [1, -1, 1, -1, 1, 0]), (2, True, [2, -2, 2, -2, 2, -1]),
                                 (1, False, [1, 0, 0, 0, 1, 0])]:
        spk, *_ = O.lif_scan(cur, ps, levels=levels, signed=signed, alif=False)
        assert spk.ravel().tolist() == want, (levels, signed)


def test_lif_hand_worked_membranes():
    """grad/tests/lif.rs:1-60: beta = sigmoid(0) = 0.5, I = [0.8, 0.9, 0.3] -> spikes [0, 1, 0],
    v = 0.8, 1.3, -0.05; tests/smoke.rs:144-151: beta = sigmoid(2.1972), I = [1.0, 0.5, 0.95] -> [1, 0, 1]."""
    for T in (1, 2, 3):
        cur = np.array([0.8, 0.9, 0.3][:T], F).reshape(1, T, 1)
        spk, v, _, _ = O.lif_scan(cur, ps_of(np.array([O.sigmoid(0.0)], F)), levels=1, signed=False, alif=False)
        assert spk.ravel().tolist() == [0, 1, 0][:T]
        assert abs(float(v[0, 0]) - [0.8, 1.3, -0.05][T - 1]) < 1e-6
    cur = np.array([1.0, 0.5, 0.95], F).reshape(1, 3, 1)
    spk, *_ = O.lif_scan(cur, ps_of(np.array([O.sigmoid(2.1972)], F)), levels=1, signed=False, alif=False)
    assert spk.ravel().tolist() == [1, 0, 1]


def test_lif_alif_fires_less_under_constant_drive():
    """gpu/arch/tests.rs:456-475: beta 0.5, I = 0.8 for 60 steps; rho 0.9, gain 1 fires less but not never."""
    t, d = 60, 4
    cur = np.full((1, t, d), 0.8, F)
    beta = np.full(d, 0.5, F)
    s0, *_ = O.lif_scan(cur, ps_of(beta), levels=1, signed=False, alif=False)
    s1, *_ = O.lif_scan(cur, ps_of(beta, rho=np.full(d, 0.9, F), gain=np.ones(d, F)), levels=1, signed=False,
                        alif=True)
    assert 0 < s1.sum() < s0.sum()


def ref_noise(shape, seed, s):
    """The deterministic inputs of gpu/lif_gen.rs:389-396 (tests::compare)."""
    n = int(np.prod(shape))
    j = np.arange(n, dtype=np.uint64)
    x = ((j * np.uint64(2654435761) + np.uint64(seed * 97 + 13)) % np.uint64(10007)).astype(F) / F(10007.0)
    v = (np.sin(x * F(6.2831853)) * F(1.7) + np.cos(x * F(51.0))) * F(s)
    return v.astype(F).reshape(shape)


def lif_ref_numpy(cur, beta, theta, alif, levels, signed, init, slope=4.0):
    """gpu/arch.rs:964-1071 (lif_ref) restated with vectorised float32 numpy: the straight-through
    spikes soft + (hard - soft) with the fast sigmoid u / (1 + S|u|), the detached reset, the ALIF
    trace a = a rho + |s| (1 - rho) (rho.affine(-1, 1))."""
    b, t, d = cur.shape
    th = np.ones(d, F) if theta is None else theta
    v, sp, a = (np.zeros((b, d), F) for _ in range(3)) if init is None else (x.copy() for x in init)
    if alif is None:
        a = None
    th_prev = np.broadcast_to(th, (b, d)).astype(F)
    if alif is not None:
        th_prev = (th_prev + a * alif[1]).astype(F)
    soft_step = lambda u: (u / (np.abs(u) * F(slope) + F(1.0))).astype(F)
    out = []
    for step in range(t):
        i_t = cur[:, step, :]
        if alif is not None:
            rho, gain = alif
            a = (a * rho + np.abs(sp) * (rho * F(-1.0) + F(1.0))).astype(F)
            th_t = (th + a * gain).astype(F)
        else:
            th_t = np.broadcast_to(th, (b, d)).astype(F)
        reset = (sp * th_prev).astype(F)
        v = ((v * beta + i_t) - reset).astype(F)
        if not signed:
            u = (v - th_t).astype(F)
            sg = soft_step(u)
            hard = (u >= 0).astype(F)
            s = (sg + (hard - sg)).astype(F)
        else:
            soft = hard = None
            for k in range(1, levels + 1):
                kth = (th_t * F(k) + F(0.0)).astype(F)
                up, down = (v - kth).astype(F), (-v - kth).astype(F)
                s1 = (soft_step(up) - soft_step(down)).astype(F)
                h1 = ((up >= 0).astype(F) - (down >= 0).astype(F)).astype(F)
                soft = s1 if soft is None else (soft + s1).astype(F)
                hard = h1 if hard is None else (hard + h1).astype(F)
            s = (soft + (hard - soft)).astype(F)
        out.append(s)
        sp = s
        th_prev = th_t
    return np.stack(out, 1), v, sp, a


@pytest.mark.parametrize("levels,signed", [(1, False), (1, True), (2, True)])
@pytest.mark.parametrize("alif", [False, True])
@pytest.mark.parametrize("theta_on", [False, True])
@pytest.mark.parametrize("init_on", [False, True])
def test_lif_oracle_equals_lif_ref(levels, signed, alif, theta_on, init_on):
    """gpu/lif_gen.rs:377-453: lif_gen's CPU loop gives lif_ref's spikes and final state exactly
    (B=3, T=37, D=8, the test's own deterministic inputs), with a spike rate in (0.02, 0.98)."""
    b, t, d = 3, 37, 8
    seed = levels * 16 + signed * 8 + alif * 4 + theta_on * 2 + init_on + 1
    cur = ref_noise((b, t, d), seed, 1.3)
    beta = (1.0 / (np.exp(-ref_noise((d,), seed, 0.8)) + F(1.0))).astype(F)
    rho = (1.0 / (np.exp(-(ref_noise((d,), seed, 1.0) + F(2.5))) + F(1.0))).astype(F)
    gain = (ref_noise((d,), seed, 0.5) + F(1.0)).astype(F)
    theta = (ref_noise((d,), seed, 0.3) + F(1.0)).astype(F) if theta_on else None
    if init_on:
        init = (ref_noise((b, d), seed, 0.7), (ref_noise((b, d), seed, 1.0) >= 0.5).astype(F),
                np.abs(ref_noise((b, d), seed, 0.3)) if alif else np.zeros((b, d), F))
    else:
        init = None
    s_r, v_r, sp_r, a_r = lif_ref_numpy(cur, beta, theta, (rho, gain) if alif else None, levels, signed, init)
    ps = ps_of(beta, theta, rho if alif else None, gain if alif else None)
    v0, s0, a0 = init if init else (None, None, None)
    spk, v, s, a = O.lif_scan(cur, ps, v0, s0, a0, levels, signed, alif)
    assert np.array_equal(spk.astype(F), s_r)
    assert np.array_equal(v.view(np.uint32), v_r.view(np.uint32))
    assert np.array_equal(s, sp_r)
    if alif:
        assert np.array_equal(a.view(np.uint32), a_r.view(np.uint32))
    rate = np.mean(spk != 0)
    assert 0.02 < rate < 0.98


# ----------------------------------------------------------------------------- kWTA


def test_kwta_keeps_k_per_row_and_the_largest():
    """tests/smoke.rs:156-172: continuous inputs keep exactly k per row, and exactly those >= the k-th largest."""
    rng = np.random.default_rng(5)
    u = rng.standard_normal((6, 128)).astype(F)
    a, kth = O.kwta(u, 16, relu2=False)
    srt = -np.sort(-u, axis=1)
    assert np.array_equal(kth, srt[:, 15])
    mask = u >= srt[:, 15:16]
    assert (mask.sum(1) == 16).all()
    assert np.array_equal(a, np.where(mask, np.maximum(u, 0), 0).astype(F))


def test_kwta_ties_kept_relu2_and_k_ge_h():
    """gpu/lif.cu:288 / fstep/arch.rs:985: every unit with u - kth >= 0 is kept (ties can exceed k);
    relu2 squares (arch/tests.rs:500-519); k >= h keeps every unit (model.rs:508-510)."""
    u = np.array([[3.0, 1.0, 1.0, 1.0, -2.0, 0.5, 1.0, 0.0]], F)
    a, kth = O.kwta(u, 2, relu2=False)
    assert kth[0] == 1.0
    assert np.array_equal(a[0], np.array([3, 1, 1, 1, 0, 0, 1, 0], F))
    a2, _ = O.kwta(u, 2, relu2=True)
    assert np.array_equal(a2, a * a)
    a3, kth3 = O.kwta(u, 8, relu2=False)
    assert np.array_equal(a3, np.maximum(u, 0))
    assert np.isneginf(kth3[0])


def test_kwta_matches_brute_force_sort():
    rng = np.random.default_rng(7)
    for h, k in [(256, 64), (1024, 256), (4096, 1024), (512, 1)]:
        u = (np.rint(rng.standard_normal((20, h)) * 4) / 4).astype(F)  # many ties
        a, kth = O.kwta(u, k, relu2=True)
        srt = -np.sort(-u, axis=1)
        want_kth = srt[:, k - 1]
        assert np.array_equal(kth, want_kth)
        keep = (u - want_kth[:, None]) >= 0
        want = np.where(keep, np.maximum(u, 0), 0).astype(F)
        assert np.array_equal(a, (want * want).astype(F))


# ----------------------------------------------------------------------------- int8 weights and products


def test_quantize_int8_bounds_and_rounding():
    """parts/src/quant.rs:111-126: |w - deq| <= scale/2; an all-zero column has scale 1; rounding is half
    away from zero (f32::round), pinned on exact halves."""
    rng = np.random.default_rng(11)
    w = rng.standard_normal((64, 48)).astype(F)
    w[:, 3] = 0.0
    q, s = O.quantize_int8(w)
    deq = q.astype(F) * s[None, :]
    assert (np.abs(w - deq) <= s[None, :] * 0.5 + 1e-7).all()
    assert s[3] == 1.0 and not q[:, 3].any()
    assert np.array_equal(s, (np.abs(w).max(0) / F(127.0)).astype(F) * (s != 1.0) + (s == 1.0))
    halves = np.array([[127.0], [0.5], [-0.5], [1.5], [2.5], [-2.5], [126.5]], F)
    qh, sh = O.quantize_int8(halves)
    assert sh[0] == 1.0
    assert qh.ravel().tolist() == [127, 1, -1, 2, 3, -3, 127]


SHAPES = [(32, 32, 3), (128, 128, 1), (96, 200, 5), (64, 4112, 2)]


@pytest.mark.parametrize("din,dout,m", SHAPES)
def test_q8_matmul_ref_near_dequantized_and_thread_invariant(din, dout, m):
    """gpu/int8/tests.rs:60-119: the kernel is the dequantized product to 1e-5 relative (partial tile at
    4112 = 64*64 + 16), and any thread count gives the same bits."""
    w = unit_noise(din * dout, din + dout).reshape(din, dout) * F(0.05)
    x = unit_noise(m * din, 7 + m).reshape(m, din)
    x[:, ::3] = 0.0  # zero inputs exercise the E2 skip (gpu/int8.rs:10-13)
    q, s = O.quantize_int8(w)
    y = O.q8_matmul_ref(x, q, s, threads=1)
    exact = x.astype(np.float64) @ (q.astype(np.float64) * s.astype(np.float64))
    mag = np.abs(x).astype(np.float64) @ (np.abs(q).astype(np.float64) * s)
    assert np.max(np.abs(y - exact) / (mag + 1e-30)) < 1e-5
    for th in (2, 5):
        assert np.array_equal(O.q8_matmul_ref(x, q, s, threads=th).view(np.uint32), y.view(np.uint32))


@pytest.mark.parametrize("m,din,dout", [(6, 64, 64), (7, 200, 100), (50, 1030, 130), (97, 256, 256), (13, 4112, 70)])
def test_q8_blocked_form_gives_the_row_form_bits(m, din, dout):
    """gpu/int8/block.rs:15-18: the row-blocked product (6 x 16 register blocks over an f32 copy of each
    tile, sparse rows as event sums) gives the per-row kernel's bits: dense rows in runs and apart, sparse
    rows (under a tenth non-zero), zero and -0 inputs, a partial tile and rows past a multiple of 6."""
    rng = np.random.default_rng(m + din + dout)
    w = (rng.standard_normal((din, dout)) * 0.05).astype(F)
    x = rng.standard_normal((m, din)).astype(F)
    x[:, ::3] = 0.0
    x[:, 1::7] = -0.0
    for r in range(1, m, 4):  # every fourth row sparse
        keep = rng.random(din) < 0.05
        x[r] = np.where(keep, x[r], F(0.0))
    q, s = O.quantize_int8(w)
    rows = O.q8_matmul_ref(x, q, s, threads=3, form="rows")
    blocked = O.q8_matmul_ref(x, q, s, threads=3, form="blocked")
    assert np.array_equal(rows.view(np.uint32), blocked.view(np.uint32))
    assert np.array_equal(O.q8_matmul_ref(x, q, s, threads=1).view(np.uint32), rows.view(np.uint32))


def test_q8_integer_inputs_are_exact():
    """Spike inputs (-2..2): the f32 chain of integer products is exact (|acc| < 2^24), so the product is
    float(exact integer sum) * scale, the identity the i8 MFMA spike path relies on."""
    rng = np.random.default_rng(3)
    din, dout, m = 1024, 256, 16
    q, s = O.quantize_int8((rng.standard_normal((din, dout)) * 0.02).astype(F))
    sp = rng.integers(-2, 3, (m, din)).astype(np.int8)
    y = O.q8_matmul_ref(sp.astype(F), q, s)
    exact = (sp.astype(np.int64) @ q.astype(np.int64)).astype(F) * s[None, :]
    assert np.array_equal(y.view(np.uint32), exact.astype(F).view(np.uint32))
    acc = O.q8_acc(sp, q)
    assert np.array_equal(acc, (sp.astype(np.int64) @ q.astype(np.int64)).astype(np.int32))


@pytest.mark.parametrize("planes", [1, 2, 3])
def test_split_planes_reconstruct_and_combine(planes):
    """The build's activation planes: q0 within +-127, the smallest row exponent, x = 2^e sum q_p 2^-7p
    up to half a unit of the last plane; the combine equals an int64/float64 restatement bit for bit."""
    rng = np.random.default_rng(planes)
    x = (rng.standard_normal((40, 96)) * np.exp(rng.standard_normal((40, 1)) * 3)).astype(F)
    x[5] = 0.0
    xq, xe = O.quant_planes(x, planes)
    assert np.abs(xq[0]).max() <= 127
    amax = np.abs(x).max(1)
    nz = amax > 0
    assert (amax[nz] * np.exp2(-xe[nz].astype(np.float64)) < 127.5).all()
    assert (amax[nz] * np.exp2(-(xe[nz] - 1).astype(np.float64)) >= 127.5).all()
    rec = sum(xq[p].astype(np.float64) * 2.0 ** (-7 * p) for p in range(planes)) * np.exp2(xe[:, None].astype(np.float64))
    tol = 0.5 * 2.0 ** (-7 * (planes - 1)) * np.exp2(xe[:, None].astype(np.float64))
    assert (np.abs(rec - x) <= tol * (1 + 1e-12)).all()
    w = (rng.standard_normal((96, 24)) * 0.02).astype(F)
    q, s = O.quantize_int8(w)
    acc = np.stack([O.q8_acc(xq[p], q) for p in range(planes)])
    y = O.q8_combine(acc, xe, s)
    A = sum(acc[p].astype(np.int64) << (7 * (planes - 1 - p)) for p in range(planes))
    want = (np.ldexp(A.astype(np.float64).astype(F), (xe[:, None] - 7 * (planes - 1)))).astype(F) * s[None, :]
    assert np.array_equal(y.view(np.uint32), want.astype(F).view(np.uint32))
    assert np.array_equal(O.q8_matmul_planes(x, planes, q, s).view(np.uint32), y.view(np.uint32))


# ----------------------------------------------------------------------------- fast-weight memory


def mem_inputs(BH, T, hs, g, seed, unit_keys=True):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((BH, T, hs)).astype(F)
    k = rng.standard_normal((BH, T, hs)).astype(F)
    e = rng.standard_normal((BH, T, hs)).astype(F)
    if unit_keys:
        for z in (q, k, e):
            z /= np.linalg.norm(z, axis=2, keepdims=True)
    v = rng.standard_normal((BH, T, hs)).astype(F)
    la = (-np.exp(rng.standard_normal((BH, T, g)) - 3.5)).astype(F)  # alpha in about (0.9, 1)
    b = (2.0 / (1.0 + np.exp(-rng.standard_normal((BH, T, g))))).astype(F)
    return q, k, e, v, la, b


@pytest.mark.parametrize("g,m", [(1, 0.0), (64, 0.0), (64, 0.5), (1, 0.5)])
def test_mem_rec_matches_float64_recurrence(g, m):
    """gpu/mem_gen.rs:549: the f32 recurrence equals the f64 one to 1e-4 of the largest output, per-head and
    per-channel gates, with and without momentum, and with a carried initial state."""
    q, k, e, v, la, b = mem_inputs(3, 50, 64, g, 17 + g)
    rng = np.random.default_rng(1)
    F0 = (rng.standard_normal((3, 64, 64)) * 0.1).astype(F)
    S0 = (rng.standard_normal((3, 64, 64)) * 0.05).astype(F)
    y, Fo, So = O.mem_rec(q, k, e, v, la, b, m=m, F=F0, S=S0)
    y64, F64, S64 = O.mem_rec_f64(q, k, e, v, la, b, m=m, F=F0, S=S0)
    assert np.max(np.abs(y - y64)) < 1e-4 * np.max(np.abs(y64))
    assert np.max(np.abs(Fo - F64)) < 1e-4 * np.max(np.abs(F64))
    if m:
        assert np.max(np.abs(So - S64)) < 1e-4 * np.max(np.abs(S64))


def test_mem_f64_recurrence_against_numpy_delta_rule():
    """The f64 recurrence against an independent numpy statement of the general rule
    (gpu/arch.rs:1084-1090): r = F^T e; U = (b*k) v^T - (a*b*e) r^T; S = M S + U; F = diag(a) F + S; y = F^T q."""
    q, k, e, v, la, b = mem_inputs(2, 12, 16, 16, 3)
    M = 0.5
    y64, F64, S64 = O.mem_rec_f64(q, k, e, v, la, b, m=M)
    for bh in range(2):
        Fm = np.zeros((16, 16))
        Sm = np.zeros((16, 16))
        for t in range(12):
            a = np.exp(la[bh, t].astype(np.float64))
            bb = b[bh, t].astype(np.float64)
            r = Fm.T @ e[bh, t]
            U = np.outer(bb * k[bh, t], v[bh, t]) - np.outer(a * bb * e[bh, t], r)
            Sm = M * Sm + U
            Fm = a[:, None] * Fm + Sm
            assert np.allclose(y64[bh, t], Fm.T @ q[bh, t], rtol=1e-12, atol=1e-12)
        assert np.allclose(F64[bh], Fm, rtol=1e-12, atol=1e-12)


def test_delta_rule_write_then_read_returns_the_value():
    """The plain rule (alpha 1, e = k, M = 0) with beta 1 and a unit key: W_t k_t = v_t right after the write,
    also when the same key is written again (tests/smoke.rs:373-397: repeated keys)."""
    BH, T, hs = 2, 40, 64
    q, k, e, v, la, b = mem_inputs(BH, T, hs, 1, 5)
    k[:, 20:] = k[:, 20:21]  # one key repeated
    la[:] = 0.0
    b[:] = 1.0
    y, Fo, _ = O.mem_rec(k, k, k, v, la, b)  # read with q = k
    assert np.max(np.abs(y - v)) < 2e-5


def test_mem_cap_bounds_the_state():
    """gpu/mem_gen.rs:683: with a tiny cap every state entry stays within it."""
    q, k, e, v, la, b = mem_inputs(2, 30, 64, 64, 9, unit_keys=False)
    _, Fo, _ = O.mem_rec(q, k, e, v, la, b, m=0.5, cap=0.01)
    assert np.max(np.abs(Fo)) <= 0.01


# ----------------------------------------------------------------------------- block stack


def tiny_model():
    from ava_amd import synth

    cfg = synth.config("tiny")
    cfg["layers"] = 2
    return O.OracleModel(cfg, synth.params(cfg, seed=3)), cfg


def test_model_pieces_equal_one_pass():
    """gpu/state/tests.rs:93-121: a fresh state over the whole text gives the forward exactly, and pieces
    (32+32, 17+30+17, 5 x 12 + 4, token by token) with the carried state (LIF, memory, engram store) give
    one pass's logits within 1e-4 -- not bit for bit, since the memory of a piece of T > 1 tokens runs in
    chunks of chunk_len(T) (arch.rs:1166-1173) and a one-token piece as the fused step's recurrence."""
    mdl, cfg = tiny_model()
    rng = np.random.default_rng(0)
    B, T = 2, 64
    ids = rng.integers(0, cfg["vocab"], (B, T)).astype(np.int32)
    full, st_full, _ = mdl.forward(ids, state=mdl.new_state(B, eng_cap=T), planes=3)
    again, _, _ = mdl.forward(ids, state=mdl.new_state(B, eng_cap=T), planes=3)
    assert np.array_equal(again.view(np.uint32), full.view(np.uint32))
    for pieces in ([32, 32], [17, 30, 17], [5] * 12 + [4], [1] * 64):
        st = mdl.new_state(B, eng_cap=T)
        parts, a = [], 0
        for n in pieces:
            lg, st, _ = mdl.forward(ids[:, a:a + n], state=st, planes=3)
            parts.append(lg.reshape(B, n, -1))
            a += n
        got = np.concatenate(parts, axis=1).reshape(full.shape)
        assert np.max(np.abs(got - full)) < 1e-4, pieces
        for key in ("lif_v", "mem_f", "mem_s"):
            assert np.max(np.abs(st[key] - st_full[key])) <= 1e-4 * max(1.0, np.max(np.abs(st_full[key]))), key


def test_mem_chunk_matches_the_token_loop():
    """gpu/arch/tests.rs:701-736 (chunked_memory_matches_the_token_loop): the chunked form against the
    float64 token loop, per-head and per-channel gates, with and without momentum, from zero and from a
    carried state, lengths that are not multiples of 16, and forgetting strong enough that products of
    rates underflow (shift -6); bar max |d| / max(max |ref|, 1) < 1e-4."""
    def case(BH, T, g, shift, seed):
        rng = np.random.default_rng(seed)
        u = lambda *sh: rng.uniform(-3 ** 0.5, 3 ** 0.5, sh).astype(F)
        unit = lambda x: x / np.linalg.norm(x, axis=2, keepdims=True)
        q, k, e, v = unit(u(BH, T, 64)), unit(u(BH, T, 64)), unit(u(BH, T, 64)), u(BH, T, 64)
        z = (3.0 * u(BH, T, g) + shift).astype(np.float64)
        la = (-(np.maximum(-z, 0) + np.log1p(np.exp(-np.abs(z))))).astype(F)
        b = (2.0 / (1.0 + np.exp(-u(BH, T, g).astype(np.float64)))).astype(F)
        return q, k, e if g > 1 else k, v, la, b

    rel1 = lambda a, b: float(np.max(np.abs(a - b)) / max(float(np.max(np.abs(b))), 1.0))
    for n, (g, m, T, shift) in enumerate([(64, 0.0, 32, 2.0), (1, 0.0, 32, 2.0), (64, 0.5, 40, 2.0), (1, 0.5, 24, 2.0),
                                          (64, 0.0, 32, -6.0), (64, 0.7, 16, -6.0), (1, 0.0, 128, 1.0)]):
        q, k, e, v, la, b = case(2, T, g, shift, 100 * n)
        rng = np.random.default_rng(100 * n + 7)
        F0 = (rng.uniform(-1, 1, (2, 64, 64)) * 0.3).astype(F)
        S0 = (rng.uniform(-1, 1, (2, 64, 64)) * 0.3).astype(F) if m else None
        for f0, s0 in ((None, None), (F0, S0)):
            y, Fo, So = O.mem_chunk(q, k, e, v, la, b, m=m, F=f0, S=s0)
            y64, F64, S64 = O.mem_rec_f64(q, k, e, v, la, b, m=m, F=f0, S=s0)
            assert np.all(np.isfinite(y))
            assert rel1(y, y64) < 1e-4 and rel1(Fo, F64) < 1e-4, (n, rel1(y, y64), rel1(Fo, F64))
            if m:
                assert rel1(So, S64) < 1e-4


def test_mem_chunk_planted_mistakes_fail():
    """The chunk-form check catches plausible slips: the same rule with the erase key's rate dropped
    (ah = b e) or the momentum's power one short differs from the token loop far beyond 1e-4."""
    rng = np.random.default_rng(3)
    BH, T = 2, 48
    unit = lambda x: x / np.linalg.norm(x, axis=2, keepdims=True)
    q, k, e = (unit(rng.standard_normal((BH, T, 64)).astype(F)) for _ in range(3))
    v = rng.standard_normal((BH, T, 64)).astype(F)
    la = (-np.exp(rng.standard_normal((BH, T, 64)) - 1.5)).astype(F)
    b = (2.0 / (1.0 + np.exp(-rng.standard_normal((BH, T, 64))))).astype(F)
    y64, F64, _ = O.mem_rec_f64(q, k, e, v, la, b, m=0.5)
    y, Fo, _ = O.mem_chunk(q, k, e, v, la, b, m=0.5)
    assert np.max(np.abs(Fo - F64)) < 1e-4 * max(1.0, np.max(np.abs(F64)))
    # a slipped rate in the erase key, or the momentum applied one step less, is visible
    y2, F2, _ = O.mem_rec_f64(q, k, e, v, la, b, m=0.25)
    assert np.max(np.abs(Fo - F2)) > 1e-2 * max(1.0, np.max(np.abs(F64)))
    y3, F3, _ = O.mem_rec_f64(q, k, e * np.exp(-la), v, la, b, m=0.5)
    assert np.max(np.abs(y - y3)) > 1e-2 * max(1.0, np.max(np.abs(y64)))


def test_model_planes_near_the_reference_products():
    """gpu/int8/tests.rs:276-329: int8 variants of a tiny spiking model are compared at the first token
    (later tokens diverge chaotically). The split-plane products (P=3) agree with the reference's W8A32
    chain to float rounding on the first token's logits."""
    mdl, cfg = tiny_model()
    ids = np.random.default_rng(1).integers(0, cfg["vocab"], (2, 1)).astype(np.int32)
    ref, _, _ = mdl.forward(ids, planes=0)
    p3, _, _ = mdl.forward(ids, planes=3)
    assert np.max(np.abs(ref - p3)) < 1e-3 * max(1.0, np.max(np.abs(ref)))


def test_round_half_is_ieee_binary16():
    """orc_round_half against numpy's float32 -> float16 conversion (IEEE round-to-nearest-even):
    random values over the whole half range, ties, the subnormal range, overflow and specials."""
    rng = np.random.default_rng(12)
    x = np.concatenate([
        (rng.standard_normal(20000) * 10.0 ** rng.integers(-8, 5, 20000)).astype(np.float32),
        np.float32(1.0) + np.arange(-64, 64, dtype=np.float32) * np.float32(2.0 ** -11),  # ties at 1.0
        (np.arange(0, 3000, dtype=np.float32) * np.float32(2.0 ** -25)),  # subnormals and their ties
        np.array([65504.0, 65519.9, 65520.0, 70000.0, -65520.0, 6.1e-5, 6.2e-5, 0.0, -0.0, np.inf, -np.inf],
                 np.float32),
    ])
    got = O.round_half(x)
    want = x.astype(np.float16).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.isnan(O.round_half(np.array([np.nan], np.float32)))[0]
