"""The backward kernels (ava_lif_scan_bwd, ava_kwta_relu2_bwd, ava_mem_scan_bwd, ava_dense_back)
against the oracle's backward (itself pinned by autograd in test_oracle_backward.py), through the
C ABI on the GPU.

Bars: the LIF backward replays the forward with the same rounding and walks back in the oracle's
order, every operation rounded alone on both sides, so it is bit-exact; so are relu²'s backward and
the dense mix's sums over blocks. The dense weights' gradients (f32 partial sums against float64) and
the memory backward (f32 on the GPU, float64 in the oracle) meet 1e-5 relative (of each output's
largest magnitude), 1e-4 over 2048 steps.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def dev(x):
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def rel(a, b):
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def lif_inputs(seed, B, T, D, levels, signed):
    rng = np.random.default_rng(seed)
    cur = (rng.normal(size=(B, T, D)) * 1.2).astype(np.float32)
    ps = np.concatenate([rng.uniform(0.15, 0.95, D), rng.uniform(0.6, 1.4, D), rng.uniform(0.8, 0.99, D),
                         rng.uniform(0.02, 0.5, D)]).astype(np.float32)
    v0 = rng.normal(size=(B, D)).astype(np.float32)
    hi = 1 if (levels == 1 or not signed) else 2
    s0 = rng.integers(0 if not signed else -hi, hi + 1, (B, D)).astype(np.float32)
    a0 = rng.uniform(0, 1, (B, D)).astype(np.float32)
    g = rng.normal(size=(B, T, D)).astype(np.float32)
    gv = rng.normal(size=(B, D)).astype(np.float32)
    ga = rng.normal(size=(B, D)).astype(np.float32)
    return cur, ps, v0, s0, a0, g, gv, ga


def run_lif(cur, ps, v0, s0, a0, g, gv, ga, levels, signed, alif, slope, rg):
    from ava_amd import ops
    st = ops.LifState(dev(v0), dev(s0), dev(a0))
    return {k: host(v) for k, v in ops.lif_gen_bwd(dev(cur), dev(ps), dev(g), init=st, g_vT=dev(gv),
                                                    g_aT=dev(ga) if alif else None, levels=levels, signed=signed,
                                                    alif=alif, slope=slope, reset_grad=rg).items()}


@pytest.mark.parametrize("T", [1, 5, 16, 77])
@pytest.mark.parametrize("levels,signed", [(2, True), (1, True), (1, False)])
@pytest.mark.parametrize("alif", [True, False])
@pytest.mark.parametrize("rg", [False, True])
@pytest.mark.parametrize("D", [40, 64])
def test_lif_bwd(T, levels, signed, alif, rg, D):
    """Segment edges: T below, at and above the 16-step segment (77 = a short first segment + 4), on a
    ragged last wave (D=40) and on whole waves of one stream (D=64)."""
    slope = 0.5 if rg else 2.0
    x = lif_inputs(T * 7 + levels + 2 * alif + 4 * rg + D, 3, T, D, levels, signed)
    print(f"lif_bwd T={T} D={D} levels={levels} signed={signed} alif={alif} rg={rg}", flush=True)
    o = O.lif_bwd(x[0], x[1], x[5], x[2], x[3], x[4], x[6], x[7] if alif else None, levels=levels, signed=signed,
                  alif=alif, slope=slope, reset_grad=rg)
    gpu = run_lif(*x, levels, signed, alif, slope, rg)
    for k in ("dI", "dv0", "dbeta") + (("da0", "drho", "dgain") if alif else ()):
        assert np.array_equal(gpu[k], o[k]), (k, rel(gpu[k], o[k]))


def test_lif_bwd_long():
    """config[1]'s sequence length and width (T 2048, D 2048) on 8 streams, int2 with ALIF and the
    reset gradient."""
    B, T, D = 8, 2048, 2048
    x = lif_inputs(5, B, T, D, 2, True)
    print(f"lif_bwd long B={B} T={T} D={D}", flush=True)
    o = O.lif_bwd(x[0], x[1], x[5], x[2], x[3], x[4], x[6], x[7], levels=2, signed=True, alif=True, slope=0.5,
                  reset_grad=True)
    gpu = run_lif(*x, 2, True, True, 0.5, True)
    for k in ("dI", "dv0", "da0", "dbeta", "drho", "dgain"):
        e = rel(gpu[k], o[k])
        print(f"  {k}: rel {e:.2e}, bit-identical {np.mean(gpu[k] == o[k]):.4f}", flush=True)
        assert np.array_equal(gpu[k], o[k]), (k, e)


def run_lif_seg(cur, ps, v0, s0, a0, g, gv, ga, levels, signed, alif, slope, rg):
    from ava_amd import ops
    st = ops.LifState(dev(v0), dev(s0), dev(a0))
    return {k: host(v) for k, v in ops.lif_gen_bwd(dev(cur), dev(ps), dev(g), init=st, g_vT=dev(gv),
                                                    g_aT=dev(ga) if alif else None, levels=levels, signed=signed,
                                                    alif=alif, slope=slope, reset_grad=rg, segments=True).items()}


@pytest.mark.parametrize("T", [1, 33, 200])
@pytest.mark.parametrize("levels,signed", [(2, True), (1, True), (1, False)])
@pytest.mark.parametrize("alif", [True, False])
@pytest.mark.parametrize("rg", [False, True])
@pytest.mark.parametrize("D", [40, 64])
def test_lif_bwd_segments(T, levels, signed, alif, rg, D):
    """ava_lif_scan_bwd_segments against the oracle's walk (which the one-lane kernel equals bit for bit):
    one step, a 32-step segment and a 1-step one, seven segments the last of them short. The segments'
    affine functions associate the backward sums differently: within 2e-6 of each output's largest
    value here. D=40 parks the states from the general scan, D=64 from the buffer-resource one."""
    slope = 0.5 if rg else 2.0
    x = lif_inputs(T * 11 + levels + 2 * alif + 4 * rg + D, 3, T, D, levels, signed)
    print(f"lif_bwd segments T={T} D={D} levels={levels} signed={signed} alif={alif} rg={rg}", flush=True)
    o = O.lif_bwd(x[0], x[1], x[5], x[2], x[3], x[4], x[6], x[7] if alif else None, levels=levels, signed=signed,
                  alif=alif, slope=slope, reset_grad=rg)
    gpu = run_lif_seg(*x, levels, signed, alif, slope, rg)
    for k in ("dI", "dv0", "dbeta") + (("da0", "drho", "dgain") if alif else ()):
        e = rel(gpu[k], o[k])
        assert e < 2e-6, (k, e)


def test_lif_bwd_segments_long():
    """The training step's shape (4 streams x 1024 channels, T 2048: 64 segments per chain), int2 with
    ALIF and the reset gradient, against the oracle's walk."""
    B, T, D = 4, 2048, 1024
    x = lif_inputs(6, B, T, D, 2, True)
    print(f"lif_bwd segments long B={B} T={T} D={D}", flush=True)
    o = O.lif_bwd(x[0], x[1], x[5], x[2], x[3], x[4], x[6], x[7], levels=2, signed=True, alif=True, slope=0.5,
                  reset_grad=True)
    gpu = run_lif_seg(*x, 2, True, True, 0.5, True)
    for k in ("dI", "dv0", "da0", "dbeta", "drho", "dgain"):
        e = rel(gpu[k], o[k])
        print(f"  {k}: rel {e:.2e}", flush=True)
        assert e < 1e-5, (k, e)


def test_kwta_relu2_bwd():
    from ava_amd import ops
    rng = np.random.default_rng(3)
    n, h, k = 2048, 4096, 1024
    u = rng.normal(size=(n, h)).astype(np.float32)
    u[:, 100:110] = u[:, 0:10]  # repeated values
    ga = rng.normal(size=(n, h)).astype(np.float32)
    a, kth = ops.kwta_relu(dev(u), k, relu2=True)
    gu = host(ops.kwta_relu2_bwd(dev(u), kth, dev(ga)))
    ref = O.kwta_relu2_bwd(u, host(kth), ga)
    assert np.array_equal(gu, ref)
    assert np.array_equal(host(kth), O.kwta(u, k)[1])  # the same threshold the oracle selects


@pytest.mark.parametrize("i", [0, 3, 7])
def test_dense_back(i):
    from ava_amd import ops
    rng = np.random.default_rng(i)
    L, M = 8, 1 << 20
    S = rng.normal(size=(L + 1, M)).astype(np.float32)
    G = rng.normal(size=(L, M)).astype(np.float32)
    wf = rng.normal(size=L * (L + 3) // 2).astype(np.float32)
    out, dw = ops.dense_back(dev(S), dev(G), dev(wf), dev(G[i]), col=i + 1, i0=i, L=L, nd=i + 2)
    ro, rdw = O.dense_back(S, G, wf, G[i], col=i + 1, i0=i, L=L, nd=i + 2)
    assert np.array_equal(host(out), ro)
    assert rel(host(dw), rdw) < 1e-5
    e, _ = ops.dense_back(dev(S), dev(G), dev(wf), dev(np.zeros(M, np.float32)), col=0, i0=0, L=L, nd=0)
    assert np.array_equal(host(e), O.dense_back(S, G, wf, np.zeros(M, np.float32), col=0, i0=0, L=L, nd=0)[0])


def mem_inputs(seed, BH, T, g, hs=64):
    rng = np.random.default_rng(seed)

    def unit(x):
        return (x / np.linalg.norm(x, axis=-1, keepdims=True)).astype(np.float32)

    q, k, e = (unit(rng.normal(size=(BH, T, hs))) for _ in range(3))
    v = rng.normal(size=(BH, T, hs)).astype(np.float32)
    la = np.log(rng.uniform(0.85, 0.999, (BH, T, g))).astype(np.float32)
    b = rng.uniform(0.1, 1.9, (BH, T, g)).astype(np.float32)
    F0 = (rng.normal(size=(BH, hs, hs)) * 0.3).astype(np.float32)
    S0 = (rng.normal(size=(BH, hs, hs)) * 0.1).astype(np.float32)
    dy = rng.normal(size=(BH, T, hs)).astype(np.float32)
    dF = (rng.normal(size=(BH, hs, hs)) * 0.2).astype(np.float32)
    dS = (rng.normal(size=(BH, hs, hs)) * 0.2).astype(np.float32)
    return q, k, e, v, la, b, F0, S0, dy, dF, dS


def run_mem(x, m, cap, init=True):
    from ava_amd import ops
    q, k, e, v, la, b, F0, S0, dy, dF, dS = x
    o = ops.mem_gen_bwd(*(dev(z) for z in (q, k, e, v, la, b, dy)), m=m, cap=cap,
                        F0=dev(F0) if init else None, S0=dev(S0) if (init and m) else None,
                        dF_T=dev(dF) if init else None, dS_T=dev(dS) if (init and m) else None)
    return {n: host(t) for n, t in o.items()}


MEM_OUT = ("dq", "dk", "de", "dv", "dla", "db", "dF0")


@pytest.mark.parametrize("T", [1, 4, 37])
@pytest.mark.parametrize("g", [64, 1])
@pytest.mark.parametrize("m", [0.0, 0.5])
@pytest.mark.parametrize("cap", [1e5, 0.6])
def test_mem_bwd(T, g, m, cap):
    """Group edges (T below, at and off the 4-step checkpoint), per-channel and per-head gates,
    momentum, and a bound that holds on many elements (cap 0.6)."""
    x = mem_inputs(T + g + int(10 * m) + int(cap < 1), 6, T, g)
    print(f"mem_bwd T={T} g={g} m={m} cap={cap}", flush=True)
    o = O.mem_rec_bwd(*x[:6], x[8], m=m, cap=cap, F0=x[6], S0=x[7] if m else None, dF_T=x[9],
                      dS_T=x[10] if m else None)
    gpu = run_mem(x, m, cap)
    for n in MEM_OUT + (("dS0",) if m else ()):
        e = rel(gpu[n], o[n])
        assert e < 1e-5, (n, e)


def test_mem_bwd_zero_state():
    x = mem_inputs(41, 4, 19, 64)
    o = O.mem_rec_bwd(*x[:6], x[8], m=0.5)
    gpu = run_mem(x, 0.5, 1e5, init=False)
    for n in MEM_OUT + ("dS0",):
        assert rel(gpu[n], o[n]) < 1e-5, n


def test_mem_bwd_long():
    """The block stack's sequence length (T 2048) with per-channel gates and momentum 0.5 on 16 heads.
    float32 against float64 over 2048 steps of a recurrence whose state decays by alpha ~ 0.85-0.999:
    the gradients meet 1e-4 relative."""
    x = mem_inputs(77, 16, 2048, 64)
    print("mem_bwd long BH=16 T=2048", flush=True)
    o = O.mem_rec_bwd(*x[:6], x[8], m=0.5, F0=x[6], S0=x[7], dF_T=x[9], dS_T=x[10])
    gpu = run_mem(x, 0.5, 1e5)
    for n in MEM_OUT + ("dS0",):
        e = rel(gpu[n], o[n])
        print(f"  {n}: rel {e:.2e}", flush=True)
        assert e < 1e-4, (n, e)


def test_mem_bwd_many_heads():
    """512 heads: one workgroup per head and 16 columns per wave (fewer heads take four workgroups per
    head, a wave's 4 columns each, and add the rows' sums of the four in a second kernel)."""
    x = mem_inputs(91, 512, 9, 64)
    print("mem_bwd BH=512 T=9", flush=True)
    o = O.mem_rec_bwd(*x[:6], x[8], m=0.5, F0=x[6], S0=x[7], dF_T=x[9], dS_T=x[10])
    gpu = run_mem(x, 0.5, 1e5)
    for n in MEM_OUT + ("dS0",):
        e = rel(gpu[n], o[n])
        assert e < 1e-5, (n, e)


def test_wrappers_ignore_the_default_dtype():
    """The wrappers allocate float32 whatever torch's default dtype is (a float64 default once gave
    float64 output buffers that the kernels, writing float32, left mostly unwritten)."""
    old = torch.get_default_dtype()
    torch.set_default_dtype(torch.float64)
    try:
        x = lif_inputs(9, 2, 3, 8, 2, True)
        o = O.lif_bwd(x[0], x[1], x[5], x[2], x[3], x[4], x[6], x[7], slope=2.0)
        gpu = run_lif(*x, 2, True, True, 2.0, False)
        for k in ("dI", "dv0", "da0", "dbeta", "drho", "dgain"):
            assert gpu[k].dtype == np.float32 and np.array_equal(gpu[k], o[k]), k
    finally:
        torch.set_default_dtype(old)
