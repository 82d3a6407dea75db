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


@pytest.mark.parametrize("g,m,T", [(1, 0.0, 37), (64, 0.0, 64), (64, 0.5, 100), (1, 0.5, 16), (64, 0.5, 1)])
def test_mem_scan_matches_recurrence(g, m, T):
    BH = 5
    print(f"mem_scan g={g} m={m} T={T}", flush=True)
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


def delta_inputs(BH, T, seed, gated):
    rng = np.random.default_rng(seed)
    q, k, v = (rng.standard_normal((BH, T, 64)).astype(np.float32) for _ in range(3))
    q /= np.linalg.norm(q, axis=2, keepdims=True)
    k /= np.linalg.norm(k, axis=2, keepdims=True)
    beta = (1.0 / (1.0 + np.exp(-rng.standard_normal((BH, T))))).astype(np.float32)  # config[2]: sigmoid(N(0,1))
    la = (-np.exp(rng.standard_normal((BH, T)) - 3.0)).astype(np.float32) if gated else np.zeros((BH, T), np.float32)
    return q, k, v, beta, la


@pytest.mark.parametrize("gated,T", [(False, 64), (False, 256), (True, 192)])
def test_delta_chunk_matches_recurrence(gated, T):
    """model.rs:744-799 vs the token loop (arch/tests.rs:704-750: chunked = recurrence within 1e-4), with a
    carried initial state; config[2]'s rule (alpha = 1, e = k, one beta per token and head, no momentum)."""
    BH = 6
    print(f"delta_chunk gated={gated} T={T}", flush=True)
    q, k, v, beta, la = delta_inputs(BH, T, 3 + T, gated)
    F0 = (np.random.default_rng(2).standard_normal((BH, 64, 64)) * 0.1).astype(np.float32)
    from ava_amd import ops
    y, F = ops.delta_rule_from(cuda(q), cuda(k), cuda(v), cuda(beta), cuda(la) if gated else None, f0=cuda(F0))
    y, F = host(y), host(F)
    g3 = lambda a: a[:, :, None]
    y64, F64, _ = O.mem_rec_f64(q, k, k, v, g3(la), g3(beta), F=F0)
    assert rel(y, y64) < 1e-4 and rel(F, F64) < 1e-4
    yo, Fo, _ = O.mem_rec(q, k, k, v, g3(la), g3(beta), F=F0)
    assert rel(y, yo) < 1e-4 and rel(F, Fo) < 1e-4


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
