"""The float64 torch statement of the training forward (tests/train_ref.py, whose autograd gradients
are the reference point of the GPU training step) against oracle/forward64.py on the same model and
decisions. The training forward is float; forward64 is the int8 model in float64. With weights that
the quantizer represents exactly (each matrix replaced by its own dequantized int8 form, the embedding
by its head's) the two models are the same, so their logits and loss must agree to rounding."""
import numpy as np
import pytest
import torch

from ava_amd import synth
from oracle import oracle as O
from oracle.forward64 import forward64

import train_ref as R

Q8 = ("win", "wout", "wq", "wk", "wv", "we", "wg", "wo", "ewq", "ewk", "ewv", "ewo", "w1", "w2")


def dequantized(prm):
    def dq(w):
        q, s = O.quantize_int8(np.ascontiguousarray(w, np.float32))
        return (q.astype(np.float32) * s[None, :]).astype(np.float32)

    out = {"tok_emb": np.ascontiguousarray(dq(np.ascontiguousarray(prm["tok_emb"].T)).T),
           "final_norm": prm["final_norm"], "blocks": []}
    for b in prm["blocks"]:
        out["blocks"].append({k: (dq(v) if k in Q8 else v) for k, v in b.items()})
    return out


@pytest.mark.parametrize("name,B,T", [("tiny", 2, 12), ("tiny_heads", 1, 9)])
def test_training_forward_matches_the_float64_stack(name, B, T):
    cfg = synth.config(name)
    prm = dequantized(synth.params(cfg, seed=71))
    rng = np.random.default_rng(72)
    ids = rng.integers(0, cfg["vocab"], (B, T)).astype(np.int32)
    tgt = rng.integers(0, cfg["vocab"], (B, T)).astype(np.int32)
    tgt[0, 0] = -1  # an ignored position
    om = O.OracleModel(cfg, prm)
    _, _, tr = om.forward(ids, state=om.new_state(B, eng_cap=T), planes=0, trace=True)
    keep = (tr["u"] - tr["kth"][:, :, None] >= 0.0).astype(np.uint8)
    dec = {"spikes": tr["spikes"], "keep": keep}
    l64, _ = forward64(cfg, prm, ids, dec)
    torch.manual_seed(0)
    P = R.leaves(prm)
    loss, logits = R.forward_t(cfg, P, ids, tgt, tr["spikes"], keep)
    lg = logits.detach().numpy()
    assert np.max(np.abs(lg - l64)) < 1e-6 * np.max(np.abs(l64))
    lp = l64 - (np.max(l64, 1, keepdims=True) + np.log(np.sum(np.exp(l64 - np.max(l64, 1, keepdims=True)), 1,
                                                                keepdims=True)))
    ok = tgt.reshape(-1) >= 0
    want = -np.mean(lp[np.nonzero(ok)[0], tgt.reshape(-1)[ok]])
    assert abs(float(loss.detach()) - want) < 1e-9 * abs(want)
    loss.backward()
    # every trained tensor gets a gradient (theta is detached and the offsets are constants)
    for i, b in enumerate(P["blocks"]):
        for k, v in b.items():
            if k in ("theta", "off") or (k == "vres" and i == 0):
                assert v.grad is None or not torch.any(v.grad != 0), (i, k)
            else:
                assert v.grad is not None and torch.any(v.grad != 0), (i, k)
