"""GPU parity of the engram read (ava_attend) against a float64 statement of the reference's
attend (model/fstep.rs:303-329: scores q.k scaled by 1/sqrt(64), softmax with the max subtracted,
the mix p.V), at store lengths that span several 1024-key chunks of the decode form and through
the tiled form for longer query blocks. Bar: 1e-5 relative to the output's magnitude (the online
softmax differs from the two-pass form only by rounding)."""
import numpy as np
import pytest
import torch

from ava_amd import ops

pytestmark = pytest.mark.gpu


def attend_f64(q, ks, vs, n0):
    B, T, _ = q.shape
    out = np.empty((B, T, 64))
    for b in range(B):
        for t in range(T):
            n = n0 + t + 1
            s = ks[b, :n].astype(np.float64) @ q[b, t].astype(np.float64) / 8.0
            p = np.exp(s - s.max())
            out[b, t] = (p / p.sum()) @ vs[b, :n].astype(np.float64)
    return out


@pytest.mark.parametrize("kv", [np.float32, np.float16])
@pytest.mark.parametrize("B,T,n0,cap", [(3, 1, 0, 8), (3, 1, 1023, 1100), (2, 1, 1024, 1100), (4, 1, 5000, 6000),
                                        (2, 3, 2047, 2100), (2, 4, 3100, 3200), (2, 70, 1500, 1600),
                                        (1, 200, 0, 200)])
def test_attend_matches_f64(B, T, n0, cap, kv):
    """f32 store, and the fp16 store (config[4]'s KV cache): the f64 statement reads the same fp16
    values, so the bar is the same."""
    print(f"attend B={B} T={T} n0={n0} cap={cap} kv={kv.__name__}", flush=True)
    rng = np.random.default_rng(B * 7 + T + n0)
    ks = rng.standard_normal((B, cap, 64)).astype(kv)
    vs = rng.standard_normal((B, cap, 64)).astype(kv)
    q = (rng.standard_normal((B, T, 64)) * 2.0).astype(np.float32)
    want = attend_f64(q, ks, vs, n0)
    got = ops.attend(torch.from_numpy(q).cuda(), torch.from_numpy(ks).cuda(), torch.from_numpy(vs).cuda(), n0)
    got = got.cpu().numpy()
    err = np.max(np.abs(got - want)) / np.max(np.abs(want))
    assert err < 1e-5, err


def test_attend_peaked_scores():
    """Large scores (one key dominates): the running max and the chunk merge keep exp from overflowing."""
    B, T, n0, cap = 2, 1, 3000, 3001
    rng = np.random.default_rng(11)
    ks = rng.standard_normal((B, cap, 64)).astype(np.float32)
    vs = rng.standard_normal((B, cap, 64)).astype(np.float32)
    q = (ks[:, [2500]] * 30.0).astype(np.float32)  # score ~ 30 * |k|^2 / 8 ~ 240 at key 2500
    want = attend_f64(q, ks, vs, n0)
    got = ops.attend(torch.from_numpy(q).cuda(), torch.from_numpy(ks).cuda(), torch.from_numpy(vs).cuda(), n0)
    got = got.cpu().numpy()
    assert np.all(np.isfinite(got))
    assert np.max(np.abs(got - want)) / np.max(np.abs(want)) < 1e-5


def attend_heads_f64(q, ks, vs, n0, heads):
    """memory::read's heads (gpu/memory.rs:610-700): head h reads dims h hd .. h hd + hd - 1 of the
    query, keys and values, scores scaled by 1/sqrt(hd)."""
    B, T, de = q.shape
    hd = de // heads
    out = np.empty((B, T, de))
    for h in range(heads):
        sl = slice(h * hd, (h + 1) * hd)
        for b in range(B):
            for t in range(T):
                n = n0 + t + 1
                s = ks[b, :n, sl].astype(np.float64) @ q[b, t, sl].astype(np.float64) / np.sqrt(hd)
                p = np.exp(s - s.max())
                out[b, t, sl] = (p / p.sum()) @ vs[b, :n, sl].astype(np.float64)
    return out


@pytest.mark.parametrize("kv", [np.float32, np.float16])
@pytest.mark.parametrize("de,heads", [(128, 4), (256, 8), (128, 2)])
@pytest.mark.parametrize("B,T,n0,cap", [(3, 1, 0, 8), (2, 1, 1030, 1100), (2, 3, 2047, 2100), (2, 70, 100, 200),
                                        (1, 130, 0, 130)])
def test_attend_heads_matches_f64(B, T, n0, cap, de, heads, kv):
    """Heads of 32 (the reference's geometry) and of 64, through the decode form (T <= 4, chunks of
    1024 keys) and the tiled form; same bar as the single head."""
    print(f"attend_heads B={B} T={T} n0={n0} cap={cap} de={de} heads={heads} kv={kv.__name__}", flush=True)
    rng = np.random.default_rng(B * 13 + T + n0 + de + heads)
    ks = rng.standard_normal((B, cap, de)).astype(kv)
    vs = rng.standard_normal((B, cap, de)).astype(kv)
    q = (rng.standard_normal((B, T, de)) * 2.0).astype(np.float32)
    want = attend_heads_f64(q, ks, vs, n0, heads)
    got = ops.attend(torch.from_numpy(q).cuda(), torch.from_numpy(ks).cuda(), torch.from_numpy(vs).cuda(), n0,
                     heads=heads).cpu().numpy()
    err = np.max(np.abs(got - want)) / np.max(np.abs(want))
    assert err < 1e-5, err
