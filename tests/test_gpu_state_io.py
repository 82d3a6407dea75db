"""A saved state resumes a conversation exactly (Model.save_state / Model.load_state, State::save /
State::load, gpu/state.rs:1225-1246): prefill, a few table-learning decode steps, save, then continue
both the live state and the restored one with the same tokens; every logit and nat of the
continuation must be the same bits. A model of other weights refuses the file."""
import numpy as np
import pytest
import torch

from ava_amd import synth

pytestmark = pytest.mark.gpu


def run(m, st, toks, nexts, t0, t1):
    """Decode toks[:, t0:t1] one token at a time, each followed by the table step on its next word."""
    out = []
    for t in range(t0, t1):
        lg = m.forward_with_state(torch.from_numpy(np.ascontiguousarray(toks[:, t:t + 1])).cuda(), st)
        nats = m.cb_learn(lg, torch.from_numpy(np.ascontiguousarray(nexts[:, t])).cuda(), st)
        torch.cuda.synchronize()
        out.append((lg.cpu().numpy(), nats.cpu().numpy()))
    return out


@pytest.mark.parametrize("half", [True, False])
def test_restored_state_continues_bit_exact(half, tmp_path):
    from ava_amd.model import Model
    B, prefill, steps, more = 3, 11, 4, 6
    print(f"state_io half={half} B={B} prefill={prefill}", flush=True)
    cfg = dict(synth.config("tiny_cb"), eng_half=half)
    prm = synth.params(cfg, seed=31)
    m = Model(cfg, prm)
    toks = np.random.default_rng(32).integers(0, cfg["vocab"], (B, prefill + steps + more)).astype(np.int32)
    nexts = np.roll(toks, -1, axis=1)
    cap = prefill + steps + more
    st = m.state(B, eng_cap=cap)
    m.forward_with_state(torch.from_numpy(np.ascontiguousarray(toks[:, :prefill])).cuda(), st)
    run(m, st, toks, nexts, prefill, prefill + steps)
    path = str(tmp_path / "conv.safetensors")
    m.save_state(st, path)
    r = m.load_state(path)
    assert (r.eng_len, r.seen, r.eng_cap) == (st.eng_len, st.seen, st.eng_cap) == (prefill + steps,) * 2 + (cap,)
    want = run(m, st, toks, nexts, prefill + steps, prefill + steps + more)
    got = run(m, r, toks, nexts, prefill + steps, prefill + steps + more)
    for i, ((wl, wn), (gl, gn)) in enumerate(zip(want, got)):
        assert np.array_equal(wl, gl), i
        assert np.array_equal(wn, gn, equal_nan=True), i
    other = Model(cfg, synth.params(cfg, seed=33))
    with pytest.raises(ValueError, match="another model"):
        other.load_state(path)
