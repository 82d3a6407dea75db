"""GPU parity of the whole block stack (ava_model_forward) against the oracle's forward.

Bars: final logits within 1e-2 absolute; fp32 membranes and fast-weight
state within 1e-4 relative; spike mismatch at most 1e-4 of units (the final spikes of every layer).
The oracle runs the same split-plane products (planes = 3) as the GPU, so the comparison isolates
the kernels; a second check against the reference's own W8A32 products bounds the first token.
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


def run_both(name, B, T, seed, layers=None, pieces=None, threads=8):
    cfg = synth.config(name)
    if layers:
        cfg["layers"] = layers
        cfg["eng_block"] = min(cfg["eng_block"], layers - 1)
    prm = synth.params(cfg, seed=seed)
    ids = np.random.default_rng(seed + 1).integers(0, cfg["vocab"], (B, T)).astype(np.int32)
    print(f"model {name} layers={cfg['layers']} B={B} T={T} seed={seed} pieces={pieces}", flush=True)
    om = O.OracleModel(cfg, prm)
    lo, so, _ = om.forward(ids, state=om.new_state(B, eng_cap=T), planes=3, threads=threads)
    from ava_amd.model import Model
    m = Model(cfg, prm)
    st = m.state(B, eng_cap=T)
    if pieces is None:
        lg = host(m.forward_with_state(torch.from_numpy(ids).cuda(), st))
    else:
        outs = []
        for a, b in pieces:
            outs.append(host(m.forward_with_state(torch.from_numpy(np.ascontiguousarray(ids[:, a:b])).cuda(), st))
                        .reshape(B, b - a, -1))
        lg = np.concatenate(outs, axis=1).reshape(B * T, -1)
    return cfg, lo, so, lg, st


def check_state(so, st):
    assert rel(host(st.lif_v), so["lif_v"]) < 1e-4
    assert rel(host(st.mem_f), so["mem_f"]) < 1e-4
    assert rel(host(st.mem_s), so["mem_s"]) < 1e-4
    s = host(st.lif_s)
    assert np.mean(s != so["lif_s"]) <= 1e-4


@pytest.mark.parametrize("B,T", [(2, 16), (3, 40)])
def test_tiny_stack_matches_oracle(B, T):
    cfg, lo, so, lg, st = run_both("tiny", B, T, seed=1)
    assert np.max(np.abs(lg - lo)) < 1e-2
    assert rel(lg, lo) < 1e-3
    check_state(so, st)
    assert st.eng_len == T


def test_stack_in_pieces_matches_one_pass():
    """gpu/state/tests.rs:106: the forward in pieces with the carried state equals one pass."""
    cfg, lo, so, lg, st = run_both("tiny", 2, 24, seed=2, pieces=[(0, 7), (7, 8), (8, 24)])
    assert np.max(np.abs(lg - lo)) < 1e-2
    check_state(so, st)


def test_config0_shape_matches_oracle():
    """config[0]'s architecture (d 512, 8 blocks, wide 2048 / k 512, engram in block 4, vocab 8192) on
    a batch of 1 with 64 prompt tokens."""
    cfg, lo, so, lg, st = run_both("ava04_d512", 1, 64, seed=3)
    assert np.max(np.abs(lg - lo)) < 1e-2
    check_state(so, st)
