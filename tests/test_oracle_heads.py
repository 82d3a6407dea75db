"""The oracle's engram read with heads (memory::read, gpu/memory.rs:610-700: d / 32 heads of 32,
scores scaled by 1/sqrt(32)), pinned without retyping it:
- a head whose output weights are zero contributes nothing, so a model of two heads of 32 whose
  second head is silenced equals a model of one head of 32 (the scale 1/sqrt(32) and each head's
  slice of the query, keys and values; the reference's W8A32 products, planes = 0);
- renaming the heads (permuting the column blocks of Wq, Wk, Wv and the row blocks of Wo together)
  leaves every logit unchanged (bit for bit with the split-plane products, whose integer sums do not
  depend on order; to rounding with the W8A32 chain): each head reads only its own slice;
- with Wk = 0 every score is 0 and each head returns the mean of its visible values, the same for
  any head count."""
import numpy as np
import pytest

from ava_amd import synth
from oracle import oracle as O


def logits(cfg, prm, ids, planes):
    om = O.OracleModel(cfg, prm)
    out, st, _ = om.forward(ids, state=om.new_state(ids.shape[0], eng_cap=ids.shape[1]), planes=planes, threads=4)
    return out, st


def setup(seed=5, B=2, T=12):
    cfg = synth.config("tiny_heads")
    prm = synth.params(cfg, seed=seed)
    ids = np.random.default_rng(seed).integers(0, cfg["vocab"], (B, T)).astype(np.int32)
    return cfg, prm, ids


def with_engram(prm, blk, **w):
    p = dict(prm)
    p["blocks"] = [dict(b) for b in prm["blocks"]]
    p["blocks"][blk].update(w)
    return p


def test_silenced_head_equals_one_head():
    cfg, prm, ids = setup()
    blk, d = cfg["eng_block"], cfg["d"]
    rng = np.random.default_rng(9)
    n = lambda *s: (rng.standard_normal(s) * 0.05).astype(np.float32)
    wq, wk, wv, wo = n(d, 32), n(d, 32), n(d, 32), n(32, d)
    one = dict(cfg, eng_dim=32, eng_heads=1)
    two = dict(cfg, eng_dim=64, eng_heads=2)
    pa = with_engram(prm, blk, ewq=wq, ewk=wk, ewv=wv, ewo=wo)
    pb = with_engram(prm, blk, ewq=np.hstack([wq, n(d, 32)]), ewk=np.hstack([wk, n(d, 32)]),
                     ewv=np.hstack([wv, n(d, 32)]), ewo=np.vstack([wo, np.zeros((32, d), np.float32)]))
    la, _ = logits(one, pa, ids, planes=0)
    lb, _ = logits(two, pb, ids, planes=0)
    assert np.array_equal(la, lb)
    # the check has teeth: the second head, unsilenced, changes the logits
    pc = with_engram(pb, blk, ewo=np.vstack([wo, n(32, d)]))
    lc, _ = logits(two, pc, ids, planes=0)
    assert not np.array_equal(la, lc)


@pytest.mark.parametrize("planes", [0, 3])
def test_renamed_heads_same_logits(planes):
    cfg, prm, ids = setup()
    blk, hd, nh = cfg["eng_block"], 32, cfg["eng_heads"]
    perm = [2, 0, 3, 1]
    cols = np.concatenate([np.arange(h * hd, (h + 1) * hd) for h in perm])
    b = prm["blocks"][blk]
    p2 = with_engram(prm, blk, ewq=np.ascontiguousarray(b["ewq"][:, cols]),
                     ewk=np.ascontiguousarray(b["ewk"][:, cols]), ewv=np.ascontiguousarray(b["ewv"][:, cols]),
                     ewo=np.ascontiguousarray(b["ewo"][cols, :]))
    la, sa = logits(cfg, prm, ids, planes)
    lb, sb = logits(cfg, p2, ids, planes)
    if planes:
        assert np.array_equal(la, lb)  # integer accumulators: the order of Wo's rows does not matter
    else:
        # the W8A32 chain adds Wo's rows in order: renamed heads change only its rounding
        assert np.max(np.abs(la - lb)) < 1e-5 * np.max(np.abs(la))
    assert np.array_equal(sa["eng_k"][:, :, cols], sb["eng_k"])
    # a swap inside one head's slice (a different function) is seen
    cols2 = cols.copy()
    cols2[[0, 1]] = cols2[[1, 0]]
    p3 = with_engram(prm, blk, ewq=np.ascontiguousarray(b["ewq"][:, cols2]),
                     ewk=np.ascontiguousarray(b["ewk"][:, cols]), ewv=np.ascontiguousarray(b["ewv"][:, cols]),
                     ewo=np.ascontiguousarray(b["ewo"][cols, :]))
    lc, _ = logits(cfg, p3, ids, planes)
    assert not np.array_equal(la, lc)


def test_zero_keys_give_the_mean_of_values_for_any_head_count():
    cfg, prm, ids = setup()
    blk, d = cfg["eng_block"], cfg["d"]
    p0 = with_engram(prm, blk, ewk=np.zeros((d, cfg["eng_dim"]), np.float32))
    outs = [logits(dict(cfg, eng_heads=h), p0, ids, planes=0)[0] for h in (1, 2, 4)]
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])
    # with keys, the head count matters
    l4, _ = logits(cfg, prm, ids, planes=0)
    l2, _ = logits(dict(cfg, eng_heads=2), prm, ids, planes=0)
    assert not np.array_equal(l4, l2)
