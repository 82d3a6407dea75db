"""GPU parity of the fast-weight memory scan (ava_mem_scan) against the oracle's recurrence.

Bar: fp32 fast-weight state and read-outs within 1e-4 relative (of the
largest magnitude), here against both the oracle's f32 loop (gpu/mem_gen.rs:220-273) and its f64
brute force.
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


def inputs(BH, T, g, seed, unit=True):
    rng = np.random.default_rng(seed)
    q, k, e, v = (rng.standard_normal((BH, T, 64)).astype(np.float32) for _ in range(4))
    if unit:
        for z in (q, k, e):
            z /= np.linalg.norm(z, axis=2, keepdims=True)
    la = (-np.exp(rng.standard_normal((BH, T, g)) - 3.5)).astype(np.float32)
    b = (2.0 / (1.0 + np.exp(-rng.standard_normal((BH, T, g))))).astype(np.float32)
    return q, k, e, v, la, b


def rel(a, b):
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


# 5 heads take four workgroups per head (columns split), 512 heads one workgroup per head
@pytest.mark.parametrize("g,m,T,BH", [(1, 0.0, 37, 5), (64, 0.0, 64, 5), (64, 0.5, 100, 5), (1, 0.5, 16, 5),
                                      (64, 0.5, 1, 5), (64, 0.5, 19, 512), (1, 0.0, 21, 512)])
def test_mem_scan_matches_recurrence(g, m, T, BH):
    print(f"mem_scan g={g} m={m} T={T} BH={BH}", flush=True)
    q, k, e, v, la, b = inputs(BH, T, g, 3 + g + T)
    rng = np.random.default_rng(7)
    F0 = (rng.standard_normal((BH, 64, 64)) * 0.1).astype(np.float32)
    S0 = (rng.standard_normal((BH, 64, 64)) * 0.05).astype(np.float32)
    from ava_amd import ops
    y, F, S = ops.mem_gen(cuda(q), cuda(k), cuda(e), cuda(v), cuda(la), cuda(b), m=m, F=cuda(F0), S=cuda(S0))
    y, F, S = host(y), host(F), host(S)
    yo, Fo, So = O.mem_rec(q, k, e, v, la, b, m=m, F=F0, S=S0)
    y64, F64, S64 = O.mem_rec_f64(q, k, e, v, la, b, m=m, F=F0, S=S0)
    assert rel(y, yo) < 1e-4 and rel(F, Fo) < 1e-4
    assert rel(y, y64) < 1e-4 and rel(F, F64) < 1e-4
    if m:
        assert rel(S, So) < 1e-4 and rel(S, S64) < 1e-4
    else:
        assert np.array_equal(S, S0)  # untouched without momentum


def test_mem_scan_cap_bounds_state():
    """gpu/mem_gen.rs:683: a tiny cap bounds every state entry (the clamp path)."""
    q, k, e, v, la, b = inputs(3, 40, 64, 11, unit=False)
    from ava_amd import ops
    y, F, S = ops.mem_gen(cuda(q), cuda(k), cuda(e), cuda(v), cuda(la), cuda(b), m=0.5, cap=0.01)
    F = host(F)
    yo, Fo, So = O.mem_rec(q, k, e, v, la, b, m=0.5, cap=0.01)
    assert np.max(np.abs(F)) <= 0.01
    assert rel(F, Fo) < 1e-4 and rel(host(y), yo) < 1e-4


def test_mem_scan_plain_rule_reads_back_values():
    """alpha 1, e = k, beta 1, unit keys: reading k right after writing (k, v) returns v."""
    q, k, e, v, la, b = inputs(4, 50, 1, 5)
    la[:] = 0.0
    b[:] = 1.0
    from ava_amd import ops
    y, _, _ = ops.mem_gen(cuda(k), cuda(k), cuda(k), cuda(v), cuda(la), cuda(b))
    assert np.max(np.abs(host(y) - v)) < 5e-5


def test_mem_scan_rejects_bad_shapes():
    from ava_amd import ops
    from ava_amd._lib import AvaError
    q = torch.zeros((2, 8, 32), device="cuda")
    la = torch.zeros((2, 8, 1), device="cuda")
    with pytest.raises(AvaError):
        ops.mem_gen(q, q, q, q, la, la)


# ----------------------------------------------------------------------------- the chunked delta rule


def delta_inputs(BH, T, seed, gated, shift=None):
    rng = np.random.default_rng(seed)
    q, k, v = (rng.standard_normal((BH, T, 64)).astype(np.float32) for _ in range(3))
    q /= np.linalg.norm(q, axis=2, keepdims=True)
    k /= np.linalg.norm(k, axis=2, keepdims=True)
    beta = (1.0 / (1.0 + np.exp(-rng.standard_normal((BH, T))))).astype(np.float32)  # config[2]: sigmoid(N(0,1))
    if not gated:
        la = np.zeros((BH, T), np.float32)
    elif shift is None:
        la = (-np.exp(rng.standard_normal((BH, T)) - 3.0)).astype(np.float32)
    else:
        # arch/tests.rs:711's gates: log sigmoid(3 N(0,1) + shift); shift -6 gives rates near 0.0025,
        # whose products over a chunk of 64 underflow float32
        z = 3.0 * rng.standard_normal((BH, T)) + shift
        la = (-(np.maximum(-z, 0.0) + np.log1p(np.exp(-np.abs(z))))).astype(np.float32)
    return q, k, v, beta, la


@pytest.mark.parametrize("gated,T,shift,ws", [(False, 64, None, True), (False, 256, None, True),
                                              (False, 256, None, False), (True, 192, None, True),
                                              (True, 128, -6.0, True), (True, 128, 2.0, True)])
def test_delta_chunk_matches_recurrence(gated, T, shift, ws):
    """model.rs:744-799 vs the token loop (arch/tests.rs:704-750: chunked = recurrence within 1e-4, including
    forgetting strong enough that products of rates underflow), with a carried initial state; config[2]'s rule
    (alpha = 1, e = k, one beta per token and head, no momentum) and its per-head gated form."""
    BH = 6
    print(f"delta_chunk gated={gated} T={T} shift={shift} workspace={ws}", flush=True)
    q, k, v, beta, la = delta_inputs(BH, T, 3 + T, gated, shift)
    if shift is not None:
        assert np.exp(la.astype(np.float64)[:, :64].sum(axis=1)).min() < 1e-38 or shift > 0
    F0 = (np.random.default_rng(2).standard_normal((BH, 64, 64)) * 0.1).astype(np.float32)
    from ava_amd import ops
    y, F = ops.delta_rule_from(cuda(q), cuda(k), cuda(v), cuda(beta), cuda(la) if gated else None, f0=cuda(F0),
                               workspace=ws)
    y, F = host(y), host(F)
    g3 = lambda a: a[:, :, None]
    y64, F64, _ = O.mem_rec_f64(q, k, k, v, g3(la), g3(beta), F=F0)
    r = rel if shift is None else rel1  # the reference's measure for its gate cases: over max(max |b|, 1)
    assert np.isfinite(y).all() and np.isfinite(F).all()
    assert r(y, y64) < 1e-4 and r(F, F64) < 1e-4
    yo, Fo, _ = O.mem_rec(q, k, k, v, g3(la), g3(beta), F=F0)
    assert r(y, yo) < 1e-4 and r(F, Fo) < 1e-4


def test_delta_chunk_repeated_keys_read_back():
    """tests/smoke.rs:373-397: two chunks, the second one key repeated; with beta 1 every read right after a
    write returns the written value (unit keys), where a power-series inverse would cancel catastrophically."""
    BH, T = 3, 128
    q, k, v, beta, la = delta_inputs(BH, T, 9, False)
    k[:, 64:] = k[:, 64:65]
    beta[:] = 1.0
    from ava_amd import ops
    y, _ = ops.delta_rule_from(cuda(k), cuda(k), cuda(v), cuda(beta))
    assert np.max(np.abs(host(y) - v)) < 1e-4


def test_delta_chunk_rejects_ragged_length():
    from ava_amd import ops
    from ava_amd._lib import AvaError
    q = torch.zeros((2, 100, 64), device="cuda")
    with pytest.raises(AvaError):
        ops.delta_rule_from(q, q, q, torch.zeros((2, 100), device="cuda"))


# ----------------------------------------------------------------------------- the chunked general memory


def chunk_case(BH, T, g, shift, seed):
    """arch/tests.rs:701-722's inputs at head size 64: unit q, k, e; log alpha = logsigmoid(3 u + shift)
    (shift -6: rates near 0.0025, products of rates underflow); b = 2 sigmoid(u); u uniform +-sqrt(3)."""
    rng = np.random.default_rng(seed)
    u = lambda *s: rng.uniform(-3 ** 0.5, 3 ** 0.5, s).astype(np.float32)
    unit = lambda x: x / np.linalg.norm(x, axis=2, keepdims=True)
    q, k, e = unit(u(BH, T, 64)), unit(u(BH, T, 64)), unit(u(BH, T, 64))
    v = u(BH, T, 64)
    z = (3.0 * u(BH, T, g) + shift).astype(np.float64)
    la = (-(np.maximum(-z, 0) + np.log1p(np.exp(-np.abs(z))))).astype(np.float32)
    b = (2.0 / (1.0 + np.exp(-u(BH, T, g).astype(np.float64)))).astype(np.float32)
    return q, k, e, v, la, b


def rel1(a, b):
    """arch/tests.rs:705-708: max |a - b| over max(max |b|, 1)."""
    return float(np.max(np.abs(a - b)) / max(float(np.max(np.abs(b))), 1.0))


@pytest.mark.parametrize("g,m,T,shift", [(64, 0.0, 32, 2.0), (1, 0.0, 32, 2.0), (64, 0.5, 40, 2.0), (1, 0.5, 24, 2.0),
                                         (64, 0.0, 32, -6.0), (64, 0.7, 16, -6.0), (1, 0.0, 128, 1.0),
                                         (64, 0.5, 5, 2.0), (64, 0.5, 2048, 3.0)])
def test_mem_chunk_matches_token_loop(g, m, T, shift):
    """arch/tests.rs:701-736 (chunked_memory_matches_the_token_loop) on the GPU: ava_mem_chunk against the
    oracle's token loop (f32 and f64) from zero and from a carried state, per-head and per-channel gates,
    with and without momentum, lengths that are not multiples of 16, strong forgetting (shift -6), and the
    stack's form (per-channel, M 0.5) over 2048 tokens. Bar: the reference's 1e-4."""
    BH = 8
    print(f"mem_chunk g={g} m={m} T={T} shift={shift}", flush=True)
    q, k, e, v, la, b = chunk_case(BH, T, g, shift, 11 + T + g)
    if g == 1:
        e = k.copy()
    rng = np.random.default_rng(5)
    init = [(None, None), ((rng.uniform(-1, 1, (BH, 64, 64)) * 0.3).astype(np.float32),
                           (rng.uniform(-1, 1, (BH, 64, 64)) * 0.3).astype(np.float32) if m else None)]
    from ava_amd import ops
    for F0, S0 in init:
        y, F, S = ops.mem_chunk(cuda(q), cuda(k), cuda(e), cuda(v), cuda(la), cuda(b), m=m,
                                F=None if F0 is None else cuda(F0), S=None if S0 is None else cuda(S0))
        y, F, S = host(y), host(F), host(S)
        assert np.all(np.isfinite(y)) and np.all(np.isfinite(F))
        for ref in (O.mem_rec(q, k, e, v, la, b, m=m, F=F0, S=S0), O.mem_rec_f64(q, k, e, v, la, b, m=m, F=F0, S=S0)):
            yo, Fo, So = ref
            assert rel1(y, yo) < 1e-4, rel1(y, yo)
            assert rel1(F, Fo) < 1e-4, rel1(F, Fo)
            if m:
                assert rel1(S, So) < 1e-4, rel1(S, So)


def test_mem_chunk_reads_back_values():
    """alpha 1, e = k, b 1, no momentum, unit keys: reading k right after writing (k, v) returns v, also
    inside a chunk (the recall solve) and across chunk ends."""
    q, k, e, v, la, b = inputs(4, 50, 1, 5)
    la[:] = 0.0
    b[:] = 1.0
    from ava_amd import ops
    y, _, _ = ops.mem_chunk(cuda(k), cuda(k), cuda(k), cuda(v), cuda(la), cuda(b))
    assert np.max(np.abs(host(y) - v)) < 5e-5


def test_mem_chunk_equals_scan_and_rejects_bad_shapes():
    """The chunked and the token-loop kernels agree (1e-4) on the general rule with a carried state; shape
    errors come back as AvaError."""
    from ava_amd import ops
    from ava_amd._lib import AvaError
    q, k, e, v, la, b = inputs(6, 300, 64, 21)
    rng = np.random.default_rng(1)
    F0 = (rng.standard_normal((6, 64, 64)) * 0.1).astype(np.float32)
    S0 = (rng.standard_normal((6, 64, 64)) * 0.05).astype(np.float32)
    a = ops.mem_chunk(*(cuda(z) for z in (q, k, e, v, la, b)), m=0.5, F=cuda(F0), S=cuda(S0))
    c = ops.mem_gen(*(cuda(z) for z in (q, k, e, v, la, b)), m=0.5, F=cuda(F0), S=cuda(S0))
    for x, z in zip(a, c):
        assert rel(host(x), host(z)) < 1e-4
    z = torch.zeros((2, 8, 32), device="cuda")
    with pytest.raises(AvaError):
        ops.mem_chunk(z, z, z, z, torch.zeros((2, 8, 1), device="cuda"), torch.zeros((2, 8, 1), device="cuda"))


def test_mem_chunk_bounds_hot_heads_per_token():
    """The bound clamp(F, +-cap) acts at every token once columns of F exceed cap / 8 at a chunk's start
    (those chunks run token by token): from a state near a small cap the chunked kernel equals the
    oracle's bounded token loop (gpu/mem_gen.rs:683), and every entry stays within the cap. Unit keys:
    with keys of norm ~8 the bounded rule is chaotic and no two summation orders agree past ~30 tokens."""
    q, k, e, v, la, b = inputs(4, 90, 64, 13, unit=True)
    rng = np.random.default_rng(4)
    cap = 0.05
    F0 = rng.uniform(-0.04, 0.04, (4, 64, 64)).astype(np.float32)
    S0 = rng.uniform(-0.02, 0.02, (4, 64, 64)).astype(np.float32)
    from ava_amd import ops
    y, F, S = ops.mem_chunk(cuda(q), cuda(k), cuda(e), cuda(v), cuda(la), cuda(b), m=0.5, cap=cap, F=cuda(F0),
                            S=cuda(S0))
    y, F, S = host(y), host(F), host(S)
    yo, Fo, So = O.mem_rec(q, k, e, v, la, b, m=0.5, cap=cap, F=F0, S=S0)
    assert np.max(np.abs(F)) <= cap
    assert np.mean(np.abs(Fo) == np.float32(cap)) > 0.05  # the bound acts
    assert rel(F, Fo) < 1e-4 and rel(y, yo) < 1e-4 and rel(S, So) < 1e-4
