"""Greedy continuations with carried state (Model.generate, generate in gpu/state.rs:1392-1458)
against the same loop over the oracle's forward: prompts of two lengths (read in separate passes),
a row that stops early (a stop rule) and leaves the batch, and the oracle's own argmax (lowest id on
ties). A token where the two disagree must be a near-tie in the oracle's logits (two ids within the
logits bar of 1e-2 of the 1e-4-level differences of summation order)."""
import numpy as np
import pytest

from ava_amd import synth
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def oracle_greedy(om, prompt, max_new, stop):
    st = om.new_state(1, eng_cap=len(prompt) + max_new)
    lg, st, _ = om.forward(np.asarray([prompt], np.int32), state=st, planes=3, threads=8)
    last, out, gaps = lg[-1], [], []
    for step in range(max_new):
        tok = int(np.argmax(last))
        srt = np.sort(last)[::-1]
        gaps.append(float(srt[0] - srt[1]))
        out.append(tok)
        if stop(out) or step + 1 == max_new:
            break
        lg, st, _ = om.forward(np.asarray([[tok]], np.int32), state=st, planes=3, threads=8)
        last = lg[-1]
    return out, gaps


def test_generate_matches_oracle_greedy():
    from ava_amd.model import Model
    cfg = synth.config("tiny")
    prm = synth.params(cfg, seed=17)
    rng = np.random.default_rng(18)
    prompts = [rng.integers(0, cfg["vocab"], n).tolist() for n in (9, 5, 9, 5)]
    stop = lambda toks: len(toks) >= 3 and toks[-1] % 7 == 0  # a row may leave early
    print(f"generate prompts={[len(p) for p in prompts]}", flush=True)
    m = Model(cfg, prm)
    got = m.generate(prompts, 10, stop=stop, batch_rows=8, eos=None)
    om = O.OracleModel(cfg, prm)
    for r, p in enumerate(prompts):
        want, gaps = oracle_greedy(om, p, 10, stop)
        if got[r] != want:
            k = next(i for i, (a, b) in enumerate(zip(got[r], want)) if a != b)
            assert gaps[k] < 1e-2, (r, k, gaps[k])
        else:
            assert len(got[r]) <= 10 and (len(got[r]) == 10 or stop(got[r]))


def test_generate_refuses_empty_prompt_and_honours_eos():
    from ava_amd.model import Model
    cfg = synth.config("tiny")
    m = Model(cfg, synth.params(cfg, seed=19))
    with pytest.raises(ValueError):
        m.generate([[1, 2], []], 4)
    first = m.generate([[3, 4, 5]], 1, eos=None)[0][0]
    assert m.generate([[3, 4, 5]], 6, eos=first) == [[]]  # eos is not included, and ends the row
    # no new tokens: empty continuations on both the device-side and the host loop
    assert m.generate([[3, 4, 5], [6, 7]], 0, eos=None) == [[], []]
    assert m.generate([[3, 4, 5]], 0) == [[]]


def test_device_side_greedy_equals_host_loop():
    """With no stop rule and no eos, the tokens stay on the device between steps; the same rows with
    a stop rule that never fires take the host loop: identical tokens, prompts of two lengths."""
    from ava_amd.model import Model
    cfg = synth.config("tiny")
    m = Model(cfg, synth.params(cfg, seed=23))
    rng = np.random.default_rng(24)
    prompts = [rng.integers(0, cfg["vocab"], n).tolist() for n in (7, 4, 7)]
    print(f"device-side greedy prompts={[len(p) for p in prompts]}", flush=True)
    dev = m.generate(prompts, 12, eos=None)
    host = m.generate(prompts, 12, eos=None, stop=lambda toks: False)
    assert dev == host and all(len(t) == 12 for t in dev)
