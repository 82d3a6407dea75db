"""GPU parity of the cerebellum head and its online table (the decode path's CB2) against the oracle.

The stream runs as the talking engine does (gpu/v51b.rs:590-611, gpu/fast4/cb.rs:25-84): a prefill, then
one token per step per stream, each step followed by the online learning step on the word that came.
Bars: logits within 1e-2 absolute; the table, its scale and the nats within
1e-4 relative; the granule codes within 1e-5 (f32 rounding of a unit-length vector).
"""
import numpy as np
import pytest
import torch

from ava_amd import synth
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def rel(a, b):
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def make(seed, readout=False, half=None):
    cfg = synth.config("tiny_cb")
    if half is not None:
        cfg["cb_half"] = half
    prm = synth.params(cfg, seed=seed)
    if readout:
        # a trained read-out cbh.wo (zero at init); scaled so the correction moves the logits
        rng = np.random.default_rng(seed + 7)
        prm["cb_w"] = (rng.standard_normal((cfg["cb_units"], cfg["d"])) * 0.05).astype(np.float32)
    from ava_amd.model import Model
    return cfg, prm, O.OracleModel(cfg, prm), Model(cfg, prm)


def run_stream(seed, B, prefill, steps, readout=False, ignore=(), half=None, scale0=None):
    cfg, prm, om, m = make(seed, readout, half)
    V = cfg["vocab"]
    toks = np.random.default_rng(seed + 1).integers(0, V, (B, prefill + steps + 1)).astype(np.int32)
    cap = prefill + steps
    print(f"cb stream seed={seed} B={B} prefill={prefill} steps={steps} readout={readout} ignore={ignore} "
          f"half={cfg['cb_half']} scale0={scale0}", flush=True)
    so = om.new_state(B, eng_cap=cap)
    st = m.state(B, eng_cap=cap)
    if scale0 is not None:
        so["cb_scale"][:] = scale0
        st.cb_scale.fill_(scale0)
    assert abs(m.cb_lr - om.cb_lr) == 0.0
    # prefill: teacher-forced over the prompt, then the online step on the word after it
    lo, so, _ = om.forward(toks[:, :prefill], state=so, planes=3, threads=8)
    lg = host(m.forward_with_state(torch.from_numpy(np.ascontiguousarray(toks[:, :prefill])).cuda(), st))
    assert np.max(np.abs(lg - lo)) < 1e-2
    assert np.max(np.abs(host(st.cb_code) - so["cb_code"])) < 1e-5
    worst = {"logits": np.max(np.abs(lg - lo))}
    last_o = lo.reshape(B, prefill, V)[:, -1]
    last_g = torch.from_numpy(lg.reshape(B, prefill, V)[:, -1].copy()).cuda()
    for t in range(steps + 1):
        nxt = toks[:, prefill + t].copy()
        for b in ignore:
            nxt[b] = -1
        no = om.cb_learn(last_o, nxt, so)
        ng = host(m.cb_learn(last_g, torch.from_numpy(nxt).cuda(), st))
        live = nxt >= 0
        assert np.all(np.isnan(ng[~live])) and np.all(np.isnan(no[~live]))
        assert rel(ng[live], no[live]) < 1e-4, (t, ng, no)
        assert rel(host(st.cb_scale), so["cb_scale"]) < 1e-12
        assert rel(host(st.cb_tab), so["cb_tab"]) < 1e-4, t
        if t == steps:
            break
        ids = toks[:, prefill + t:prefill + t + 1]
        lo, so, _ = om.forward(ids, state=so, planes=3, threads=8)
        lgt = m.forward_with_state(torch.from_numpy(np.ascontiguousarray(ids)).cuda(), st)
        lg = host(lgt)
        worst["logits"] = max(worst["logits"], np.max(np.abs(lg - lo)))
        assert np.max(np.abs(lg - lo)) < 1e-2, t
        assert np.max(np.abs(host(st.cb_code) - so["cb_code"])) < 1e-5
        last_o, last_g = lo, lgt
    print("worst", worst, flush=True)
    return cfg, so, st


def test_cb_prefill_then_decode_with_online_table():
    run_stream(seed=1, B=3, prefill=8, steps=6)


def test_cb_readout_and_ignored_streams():
    """A nonzero read-out W and one stream whose next word is outside the vocabulary (IGNORE: its table
    and scale stay as they are)."""
    cfg, so, st = run_stream(seed=2, B=4, prefill=5, steps=4, readout=True, ignore=(2,))
    assert host(st.cb_scale)[2] == 1.0


def test_cb_scale_fold():
    """The scale starts just above 1e-18 so the first step folds it into the table (gpu/v51b.rs:352-367)."""
    cfg, so, st = run_stream(seed=3, B=2, prefill=4, steps=2, half=2.0, scale0=1.2e-18)
    assert np.all(host(st.cb_scale) > 0.5)


def test_cb_large_code_width():
    """config[4]'s granule width (12,288 units, 384 kept) over d = 1024 inputs on a short stream: the
    code of the stack's final state through the wide top-k path."""
    cfg = synth.config("ava04_d1024_decode")
    cfg.update(layers=1, eng_block=0, vocab=512, hidden=1024, kwta_k=256)
    prm = synth.params(cfg, seed=4)
    from ava_amd.model import Model
    om, m = O.OracleModel(cfg, prm), Model(cfg, prm)
    B, T = 2, 3
    ids = np.random.default_rng(5).integers(0, cfg["vocab"], (B, T)).astype(np.int32)
    print(f"cb wide B={B} T={T} G={cfg['cb_units']}", flush=True)
    so, st = om.new_state(B, eng_cap=T), m.state(B, eng_cap=T)
    lo, so, _ = om.forward(ids, state=so, planes=3, threads=8)
    lg = host(m.forward_with_state(torch.from_numpy(ids).cuda(), st))
    assert np.max(np.abs(lg - lo)) < 1e-2
    c = host(st.cb_code)
    assert np.max(np.abs(c - so["cb_code"])) < 1e-5
    assert np.all((c != 0).sum(1) <= cfg["cb_units"] // 32)
    nxt = np.array([1, 7], np.int32)
    no = om.cb_learn(lo.reshape(B, T, -1)[:, -1], nxt, so)
    ng = host(m.cb_learn(torch.from_numpy(lg.reshape(B, T, -1)[:, -1].copy()).cuda(), torch.from_numpy(nxt).cuda(),
                         st))
    assert rel(ng, no) < 1e-4
    assert rel(host(st.cb_tab), so["cb_tab"]) < 1e-4
