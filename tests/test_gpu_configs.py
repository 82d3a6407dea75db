"""BASELINE.json's standalone configs at their full workloads, through the C ABI, against the oracle.

config[1]: the LIF scan at B=64, T=2048, C=2048 on the kernel the library picks for that size (the
one bench.py times): spikes, v_T, a_T and theta_T bit for bit (gpu/lif_gen.rs:379-453 asserts exact
spikes and state).
config[2]: the plain delta rule at B=32, H=8, T=4096, d=64 in chunks of 64 against the f64
recurrence (gpu/mem_gen.rs:220-273 with alpha = 1, e = k, one beta per head, no momentum): read-outs
and final state within 1e-4 relative of the largest magnitude (north_star's fp32-state bar; the
chunked form against the recurrence is pinned to 1e-4 by gpu/arch/tests.rs:704-750).
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


def rel(a, b):
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def sig(x):
    return (1.0 / (np.exp(-np.asarray(x, np.float32)) + np.float32(1.0))).astype(np.float32)


def test_config1_lif_full_size_bit_exact(dev):
    """config[1] in full: cur ~N(0,1) [64, 2048, 2048]; beta = sigmoid(U(1.5, 4.5)); theta 1, ALIF
    rho 0.95 and gain 0.05; int2 spikes with subtract reset."""
    from ava_amd import ops
    B, T, D = 64, 2048, 2048
    rng = np.random.default_rng(101)
    cur = rng.standard_normal((B, T, D), dtype=np.float32)
    beta = sig(rng.uniform(1.5, 4.5, D))
    ps = np.concatenate([beta, np.ones(D, np.float32), np.full(D, 0.95, np.float32),
                         np.full(D, 0.05, np.float32)]).astype(np.float32)
    print(f"config[1] LIF B={B} T={T} D={D}: GPU scan", flush=True)
    spk, st, th = ops.lif_gen(cuda(cur), cuda(beta), cuda(ps[D:2 * D]), (cuda(ps[2 * D:3 * D]), cuda(ps[3 * D:])),
                              levels=2, signed=True, th_out=True)
    spk_g, v_g, a_g, th_g = host(spk), host(st.v), host(st.a), host(th)
    del spk, st, th
    print("config[1] LIF: oracle scan", flush=True)
    spk_o, v_o, s_o, a_o = O.lif_scan(cur, ps, levels=2, signed=True, alif=True)
    assert np.array_equal(spk_g, spk_o)
    assert np.array_equal(v_g.view(np.uint32), v_o.view(np.uint32))
    assert np.array_equal(a_g.view(np.uint32), a_o.view(np.uint32))
    th_o = (ps[D:2 * D][None, :] + a_o * ps[3 * D:][None, :]).astype(np.float32)
    assert np.array_equal(th_g.view(np.uint32), th_o.view(np.uint32))
    counts = np.bincount((spk_o.reshape(-1).astype(np.int16) + 2), minlength=5)
    print("spike counts -2..2:", counts.tolist(), flush=True)
    assert counts[0] > 0 and counts[4] > 0  # both levels occur on both sides


def test_config2_delta_rule_full_size(dev):
    """config[2] in full: q, k L2-normalised N(0,1); v N(0,1); beta = sigmoid(N(0,1)) per token and
    head; W_0 = 0; chunks of 64."""
    from ava_amd import ops
    Bn, H, T, hs = 32, 8, 4096, 64
    BH = Bn * H
    rng = np.random.default_rng(202)
    q = rng.standard_normal((BH, T, hs), dtype=np.float32)
    k = rng.standard_normal((BH, T, hs), dtype=np.float32)
    q /= np.linalg.norm(q, axis=2, keepdims=True)
    k /= np.linalg.norm(k, axis=2, keepdims=True)
    v = rng.standard_normal((BH, T, hs), dtype=np.float32)
    beta = sig(rng.standard_normal((BH, T)))
    print(f"config[2] delta rule BH={BH} T={T}: GPU chunked form", flush=True)
    y, F = ops.delta_rule_from(cuda(q), cuda(k), cuda(v), cuda(beta))
    y, F = host(y), host(F)
    print("config[2] delta rule: oracle f64 recurrence", flush=True)
    la = np.zeros((BH, T, 1), np.float32)
    y64, F64, _ = O.mem_rec_f64(q, k, k, v, la, beta[:, :, None])
    ry, rF = rel(y, y64), rel(F, F64)
    print(f"rel y {ry:.2e}  rel F {rF:.2e}", flush=True)
    assert ry < 1e-4 and rF < 1e-4
