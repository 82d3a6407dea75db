"""GPU parity of the single ops (LIF scan, kWTA, int8 weights/planes/products) against the oracle.

Bars: int8 accumulators, kWTA index sets and LIF spikes/state are
bit-exact; f32 products within the stated tolerance.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def cuda(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


# ----------------------------------------------------------------------------- LIF


def ref_noise(shape, seed, s):
    """The deterministic inputs of lif_gen.rs:389-396 (tests::compare)."""
    n = int(np.prod(shape))
    j = np.arange(n, dtype=np.uint64)
    x = ((j * np.uint64(2654435761) + np.uint64(seed * 97 + 13)) % np.uint64(10007)).astype(np.float32) / np.float32(10007.0)
    v = (np.sin(x * np.float32(6.2831853)) * np.float32(1.7) + np.cos(x * np.float32(51.0))) * np.float32(s)
    return v.astype(np.float32).reshape(shape)


def sig(x):
    return (1.0 / (np.exp(-x.astype(np.float32)) + np.float32(1.0))).astype(np.float32)


@pytest.mark.parametrize("levels,signed", [(1, False), (1, True), (2, True)])
@pytest.mark.parametrize("alif", [False, True])
@pytest.mark.parametrize("theta_on", [False, True])
@pytest.mark.parametrize("init_on", [False, True])
@pytest.mark.parametrize("d", [8, 64])
def test_lif_matches_oracle_every_option(levels, signed, alif, theta_on, init_on, d, dev):
    """lif_gen.rs:377-453: every option, spikes and final state exactly (B=3, T=37: one 32-step block
    and a ragged tail). D=8 takes the general scan, D=64 the buffer-resource one (D a multiple of 64)."""
    b, t = 3, 37
    seed = levels * 16 + signed * 8 + alif * 4 + theta_on * 2 + init_on + 1 + d
    cur = ref_noise((b, t, d), seed, 1.3)
    beta = sig(ref_noise((d,), seed, 0.8))
    rho = sig(ref_noise((d,), seed, 1.0) + np.float32(2.5))
    gain = ref_noise((d,), seed, 0.5) + np.float32(1.0)
    theta = ref_noise((d,), seed, 0.3) + np.float32(1.0) if theta_on else np.ones(d, np.float32)
    ps = np.concatenate([beta, theta, rho if alif else np.zeros(d, np.float32),
                         gain if alif else np.zeros(d, np.float32)]).astype(np.float32)
    if init_on:
        v0 = ref_noise((b, d), seed, 0.7)
        a0 = np.abs(ref_noise((b, d), seed, 0.3)) if alif else np.zeros((b, d), np.float32)
        s0 = (ref_noise((b, d), seed, 1.0) >= 0.5).astype(np.float32)
    else:
        v0 = s0 = a0 = np.zeros((b, d), np.float32)
    spk_o, v_o, s_o, a_o = O.lif_scan(cur, ps, v0, s0, a0, levels, signed, alif)
    from ava_amd import ops
    init = ops.LifState(cuda(v0), cuda(s0), cuda(a0))
    spk, st = ops.lif_gen(cuda(cur), cuda(beta), cuda(theta), (cuda(ps[2 * d:3 * d]), cuda(ps[3 * d:])) if alif else None,
                          levels=levels, signed=signed, init=init)
    assert np.array_equal(host(spk), spk_o)
    assert np.array_equal(host(st.v).view(np.uint32), v_o.view(np.uint32))
    assert np.array_equal(host(st.s), s_o)
    assert np.array_equal(host(st.a).view(np.uint32), a_o.view(np.uint32))
    rate = np.mean(spk_o != 0)
    assert 0.02 < rate < 0.98


@pytest.mark.parametrize("B,T,D", [(4, 300, 256), (3, 31, 200), (1, 65, 64)])
def test_lif_config1_shape_bit_exact(B, T, D, dev):
    """config[1] semantics (int2, ALIF rho 0.95 gain 0.05, theta 1, beta = sigmoid(U(1.5, 4.5))) on a
    reduced batch, with T shorter than, equal to and past the steps in flight and a partial workgroup:
    spikes, v_T, a_T and theta_T bit for bit."""
    rng = np.random.default_rng(11)
    cur = rng.standard_normal((B, T, D), dtype=np.float32)
    beta = sig(rng.uniform(1.5, 4.5, D).astype(np.float32))
    ps = np.concatenate([beta, np.ones(D, np.float32), np.full(D, 0.95, np.float32),
                         np.full(D, 0.05, np.float32)]).astype(np.float32)
    spk_o, v_o, s_o, a_o = O.lif_scan(cur, ps, levels=2, signed=True, alif=True)
    from ava_amd import ops
    spk, st, th = ops.lif_gen(cuda(cur), cuda(beta), cuda(ps[D:2 * D]), (cuda(ps[2 * D:3 * D]), cuda(ps[3 * D:])),
                              levels=2, signed=True, th_out=True)
    assert np.array_equal(host(spk), spk_o)
    assert np.array_equal(host(st.v).view(np.uint32), v_o.view(np.uint32))
    assert np.array_equal(host(st.a).view(np.uint32), a_o.view(np.uint32))
    th_o = (ps[D:2 * D][None, :] + a_o * ps[3 * D:][None, :]).astype(np.float32)
    assert np.array_equal(host(th).view(np.uint32), th_o.view(np.uint32))
    assert np.mean(np.abs(spk_o) == 2) > 0  # both levels occur


# ----------------------------------------------------------------------------- kWTA


def kwta_cases():
    rng = np.random.default_rng(5)
    yield "reference 6x128 k16", rng.standard_normal((6, 128)).astype(np.float32), 16
    yield "config3 rows", rng.standard_normal((64, 4096)).astype(np.float32), 1024
    yield "config0 rows", rng.standard_normal((33, 2048)).astype(np.float32), 512
    ties = (np.rint(rng.standard_normal((40, 1024)) * 2) / 2).astype(np.float32)
    yield "heavy ties", ties, 256
    yield "all negative", -np.abs(rng.standard_normal((8, 512))).astype(np.float32) - 0.1, 64
    yield "k >= h", rng.standard_normal((5, 256)).astype(np.float32), 256
    yield "k = 1", rng.standard_normal((7, 256)).astype(np.float32), 1
    yield "wide 8192", rng.standard_normal((3, 8192)).astype(np.float32), 2048


@pytest.mark.parametrize("relu2", [False, True])
def test_kwta_matches_oracle(relu2, dev):
    from ava_amd import ops
    for name, u, k in kwta_cases():
        a_o, kth_o = O.kwta(u, k, relu2)
        a, kth = ops.kwta_relu(cuda(u), k, relu2)
        a, kth = host(a), host(kth)
        assert np.array_equal(a.view(np.uint32) != 0, a_o.view(np.uint32) != 0) or np.array_equal(a != 0, a_o != 0), name
        assert np.array_equal(a, a_o), name
        if k < u.shape[1]:
            assert np.array_equal(kth, kth_o), name
            # the index set: every kept unit is >= kth, at least k per row
            assert (np.sum(u - kth[:, None] >= 0, axis=1) >= k).all(), name


# ----------------------------------------------------------------------------- int8 products

# m <= 512 takes the few-rows kernel (32 x 32 blocks, K steps over the waves), larger m the tiled ones;
# the last shape has more 128 x 256 tiles (65 x 5, edge tiles in both directions) than an MI355X has
# CUs, so workgroups of the persistent grid take several tiles each
SHAPES = [(32, 32, 3), (128, 128, 1), (96, 200, 5), (64, 4112, 2), (1024, 1024, 300), (1024, 192, 129),
          (4096, 1024, 257), (1024, 1024, 700), (512, 4112, 530), (256, 1100, 8300)]


@pytest.mark.parametrize("din,dout,m", SHAPES)
def test_q8_pack_matches_quantizer(din, dout, m, dev):
    rng = np.random.default_rng(din + dout)
    w = (rng.standard_normal((din, dout)) * 0.02).astype(np.float32)
    w[:, 0] = 0.0  # an all-zero column: scale 1
    q_o, s_o = O.quantize_int8(w)
    from ava_amd import ops
    qw = ops.QW.from_tensor(cuda(w))
    qt, sc = host(qw.qt), host(qw.scale)
    assert np.array_equal(sc.view(np.uint32), s_o.view(np.uint32))
    assert np.array_equal(qt[:, :din], q_o.T)
    assert not qt[:, din:].any()
    assert sc[0] == 1.0


@pytest.mark.parametrize("planes", [1, 2, 3])
def test_quant_rows_matches_oracle(planes, dev):
    rng = np.random.default_rng(planes)
    x = (rng.standard_normal((67, 200)) * np.exp(rng.standard_normal((67, 1)) * 3)).astype(np.float32)
    x[3] = 0.0
    x[4, :5] = 127.49
    xq_o, xe_o = O.quant_planes(x, planes)
    from ava_amd import ops
    xq, xe = ops.quant_rows(cuda(x), planes)
    xq, xe = host(xq), host(xe)
    assert np.array_equal(xe, xe_o)
    assert np.array_equal(xq[:, :, :200], xq_o)
    assert not xq[:, :, 200:].any()


@pytest.mark.parametrize("din,dout,m", SHAPES)
def test_q8_accumulators_bit_exact(din, dout, m, dev):
    rng = np.random.default_rng(din * 7 + m)
    w = (rng.standard_normal((din, dout)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, din)).astype(np.float32)
    q_o, s_o = O.quantize_int8(w)
    xq_o, xe_o = O.quant_planes(x, 3)
    from ava_amd import ops
    qw = ops.QW.from_tensor(cuda(w))
    xq, _ = ops.quant_rows(cuda(x), 3)
    acc = host(ops.gemm_acc(xq, qw))
    for p in range(3):
        assert np.array_equal(acc[p], O.q8_acc(xq_o[p], q_o)), f"plane {p}"


@pytest.mark.parametrize("din,dout,m", SHAPES)
def test_q8_matmul_planes_bit_exact_and_near_f32(din, dout, m, dev):
    rng = np.random.default_rng(din + 3 * m)
    w = (rng.standard_normal((din, dout)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, din)).astype(np.float32)
    q_o, s_o = O.quantize_int8(w)
    from ava_amd import ops
    qw = ops.QW.from_tensor(cuda(w))
    y = host(ops.mm(cuda(x), qw, planes=3))
    assert np.array_equal(y.view(np.uint32), O.q8_matmul_planes(x, 3, q_o, s_o).view(np.uint32))
    # against the dequantized product in f64, and the reference's W8A32 chain (int8/tests.rs:60-89: 1e-5)
    exact = x.astype(np.float64) @ (q_o.astype(np.float64) * s_o.astype(np.float64))
    ref = O.q8_matmul_ref(x, q_o, s_o)
    scale = np.abs(x).astype(np.float64) @ (np.abs(q_o).astype(np.float64) * s_o)
    assert np.max(np.abs(y - exact) / (scale + 1e-30)) < 1e-5
    assert np.max(np.abs(ref - exact) / (scale + 1e-30)) < 1e-5


@pytest.mark.parametrize("din,dout,m", [(1024, 512, 600), (4096, 512, 600), (2048, 300, 530)])
@pytest.mark.parametrize("planes", [2, 3])
def test_q8_tiled_plane_combines_bit_exact(din, dout, m, planes, dev):
    """The tiled product's two exact plane combinations, against the oracle's bits: K <= 1024 adds the top
    two planes in int32 first, longer K combines every plane in double (2048 x 300: edge tiles in both
    directions). Rows spread over 40 binades so the row exponents differ."""
    rng = np.random.default_rng(din + dout + m + planes)
    w = (rng.standard_normal((din, dout)) * 0.02).astype(np.float32)
    x = (rng.standard_normal((m, din)) * np.exp2(rng.integers(-20, 20, (m, 1)))).astype(np.float32)
    q_o, s_o = O.quantize_int8(w)
    from ava_amd import ops
    qw = ops.QW.from_tensor(cuda(w))
    y = host(ops.mm(cuda(x), qw, planes=planes))
    assert np.array_equal(y.view(np.uint32), O.q8_matmul_planes(x, planes, q_o, s_o).view(np.uint32))


@pytest.mark.parametrize("din,dout,m", [(1024, 512, 600), (4096, 512, 600), (1024, 1100, 300), (2048, 300, 530)])
@pytest.mark.parametrize("kind", [2, 3])
def test_q8_epilogues_scale_and_accumulate_bit_exact(din, dout, m, kind, dev):
    """The stack's two other product epilogues through the library's own ava::q8_gemm: kind 2 stores
    v * colv[col], kind 3 adds v to the prior y, each one f32 rounding after the oracle's product v, on
    the tiled kernel (both plane combinations, edge tiles) and the few-rows one (300 rows)."""
    import ctypes as C
    import torch
    from ava_amd import ops, _lib
    f = getattr(_lib.lib(), "_ZN3ava7q8_gemmEPKaPKiiiPK6ava_qwiPfiPKfP12ihipStream_t")
    f.restype = C.c_int
    f.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_void_p,
                  C.c_void_p]
    rng = np.random.default_rng(din + dout + m + kind)
    w = (rng.standard_normal((din, dout)) * 0.02).astype(np.float32)
    x = (rng.standard_normal((m, din)) * np.exp2(rng.integers(-8, 8, (m, 1)))).astype(np.float32)
    y0 = rng.standard_normal((m, dout)).astype(np.float32)
    cv = rng.uniform(0.5, 2.0, dout).astype(np.float32)
    q_o, s_o = O.quantize_int8(w)
    v = O.q8_matmul_planes(x, 3, q_o, s_o)
    want = (v * cv).astype(np.float32) if kind == 2 else (y0 + v).astype(np.float32)
    qw = ops.QW.from_tensor(cuda(w))
    xq, xe = ops.quant_rows(cuda(x), 3)
    y = cuda(y0)
    colv = cuda(cv)
    rc = f(xq.data_ptr(), xe.data_ptr(), 3, m, C.addressof(qw.c), kind, y.data_ptr(), dout, colv.data_ptr(),
           torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    assert np.array_equal(host(y).view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("din,dout,m", SHAPES)
def test_q8_spike_product_is_the_reference_bits(din, dout, m, dev):
    """Integer inputs: the i8 MFMA product equals the reference's f32 fma chain bit for bit."""
    rng = np.random.default_rng(din + dout + m)
    w = (rng.standard_normal((din, dout)) * 0.02).astype(np.float32)
    s = rng.integers(-2, 3, (m, din)).astype(np.int8)
    s[rng.random((m, din)) < 0.8] = 0
    q_o, s_o = O.quantize_int8(w)
    from ava_amd import ops
    qw = ops.QW.from_tensor(cuda(w))
    sp = np.zeros((m, qw.ldk), np.int8)
    sp[:, :din] = s
    y = host(ops.mm_spikes(cuda(sp), qw))
    ref = O.q8_matmul_ref(s.astype(np.float32), q_o, s_o)
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))
