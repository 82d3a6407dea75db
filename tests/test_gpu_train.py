"""The float32 training step (ava_train_step) against autograd of the float64 torch statement of the
same forward (tests/train_ref.py, pinned against oracle/forward64.py in tests/test_train_ref.py),
with the GPU step's own spikes and kWTA index sets forced in the statement. Bars: the loss within 1e-5
relative, every parameter's gradient within 1e-4 of that tensor's largest reference magnitude."""
import numpy as np
import pytest
import torch

from ava_amd import synth

import train_ref as R

pytestmark = pytest.mark.gpu


def rel(a, b):
    return float(np.max(np.abs(np.asarray(a, np.float64) - b)) / max(np.max(np.abs(b)), 1e-30))


# T 45 and 70 take the attention's backward over several 32-token tiles with a ragged last one; T 200
# (from 128 steps, with few chains) the LIF backward in parallel segments, the last one short
@pytest.mark.parametrize("name,B,T", [("tiny", 2, 16), ("tiny_heads", 2, 12), ("small", 1, 24), ("tiny", 1, 45),
                                      ("tiny_heads", 1, 70), ("tiny", 2, 200)])
def test_train_step_matches_autograd(name, B, T):
    from ava_amd.train import Trainer
    cfg = synth.config(name)
    prm = synth.params(cfg, seed=81)
    rng = np.random.default_rng(82)
    ids = rng.integers(0, cfg["vocab"], (B, T)).astype(np.int32)
    tgt = rng.integers(0, cfg["vocab"], (B, T)).astype(np.int32)
    tgt[-1, 3] = -1  # a position that does not count
    print(f"train step {name} B={B} T={T}", flush=True)
    tr = Trainer(cfg, slope=4.0)
    flat = tr.pack(prm)
    loss, grads = tr.step(flat, torch.from_numpy(ids).cuda(), torch.from_numpy(tgt).cuda())
    torch.cuda.synchronize()
    dec = tr.decisions(B, T)
    spikes = dec["spikes"].cpu().numpy()
    keep = (dec["u"] - dec["kth"][:, :, None] >= 0.0).to(torch.uint8).cpu().numpy()
    assert 0.0 < np.mean(spikes != 0) < 0.6
    lr, _, gr = R.grads_t(cfg, prm, ids, tgt, spikes, keep, slope=4.0)
    lg = float(loss.item())
    print(f"{name}: loss {lg:.6f} against {lr:.6f}", flush=True)
    assert abs(lg - lr) < 1e-5 * abs(lr)
    g = tr.unpack(grads)
    worst = ("", 0.0)
    for nm in ("tok_emb", "final_norm"):
        e = rel(g[nm].cpu().numpy(), gr[nm])
        worst = max(worst, (nm, e), key=lambda z: z[1])
        assert e < 1e-4, (nm, e)
    for i, b in enumerate(gr["blocks"]):
        for nm, want in b.items():
            got = g["blocks"][i][nm].cpu().numpy()
            if not np.any(want):
                assert not np.any(got), (i, nm)  # theta, the offsets, block 0's vres
                continue
            e = rel(got, want)
            worst = max(worst, (f"{nm}[{i}]", e), key=lambda z: z[1])
            assert e < 1e-4, (i, nm, e)
    print(f"{name}: largest gradient difference {worst[1]:.2e} ({worst[0]})", flush=True)


def test_train_step_repeats_and_changes_with_the_batch():
    """Two steps on the same batch give the same loss and gradients up to the embedding's atomic adds; a
    different batch size reallocates and still matches its own first call."""
    from ava_amd.train import Trainer
    cfg = synth.config("tiny")
    prm = synth.params(cfg, seed=83)
    tr = Trainer(cfg)
    flat = tr.pack(prm)
    rng = np.random.default_rng(84)
    for B, T in ((2, 8), (3, 5), (2, 8)):
        ids = torch.from_numpy(rng.integers(0, cfg["vocab"], (B, T)).astype(np.int32)).cuda()
        tgt = torch.from_numpy(rng.integers(0, cfg["vocab"], (B, T)).astype(np.int32)).cuda()
        l1, g1 = tr.step(flat, ids, tgt)
        l1, g1 = l1.clone(), g1.clone()
        l2, g2 = tr.step(flat, ids, tgt)
        torch.cuda.synchronize()
        assert float(l1) == float(l2)
        assert torch.allclose(g1, g2, rtol=0, atol=1e-6 * float(g1.abs().max()))
