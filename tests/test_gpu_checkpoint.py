"""A model built from a file in the reference's naming (Model.from_safetensors) runs the same
forward as the model built from the same arrays: the same logits, bit for bit."""
import numpy as np
import pytest
import torch

from ava_amd import checkpoint as ck
from ava_amd import synth

pytestmark = pytest.mark.gpu


def test_model_from_safetensors_equals_model_from_arrays(tmp_path):
    from ava_amd.model import Model
    cfg = synth.config("tiny_cb")
    prm = synth.params(cfg, seed=9)
    path = str(tmp_path / "m.safetensors")
    ck.save_safetensors(path, cfg, prm)
    print(f"checkpoint tiny_cb {path}", flush=True)
    ids = torch.from_numpy(np.random.default_rng(2).integers(0, cfg["vocab"], (2, 12)).astype(np.int32)).cuda()
    a = Model(cfg, prm)
    b = Model.from_safetensors(path, ck.arch_of(cfg), cb_eta=cfg["cb_eta"], cb_half=cfg["cb_half"])
    la, _ = a.forward(ids)
    lb, _ = b.forward(ids)
    torch.cuda.synchronize()
    assert np.array_equal(la.cpu().numpy(), lb.cpu().numpy())


@pytest.mark.parametrize("name", ["tiny_heads", "tiny_cb"])
def test_model_from_safetensors_matches_oracle(name, tmp_path):
    """The file read back with its recipe found beside it (NAME.arch.txt, gpu/ckpt.rs:97-112) and its
    engram heads from the file, against the oracle built from the loaded arrays: logits within 1e-2
    absolute and 1e-3 relative."""
    from ava_amd.model import Model
    from oracle import oracle as O
    cfg = synth.config(name)
    prm = synth.params(cfg, seed=19)
    path = str(tmp_path / "m.safetensors")
    ck.save_safetensors(path, cfg, prm, write_arch=True)
    over = dict(cb_eta=cfg["cb_eta"], cb_half=cfg["cb_half"]) if cfg.get("cb_units") else {}
    cfg2, prm2 = ck.load_safetensors(path, **over)
    assert max(1, cfg2["eng_heads"]) == max(1, cfg.get("eng_heads", 1) or 1)
    B, T = 2, 12
    ids = np.random.default_rng(3).integers(0, cfg["vocab"], (B, T)).astype(np.int32)
    print(f"checkpoint {name} vs oracle B={B} T={T}", flush=True)
    m = Model.from_safetensors(path, **over)
    lg = m.forward_with_state(torch.from_numpy(ids).cuda(), m.state(B, eng_cap=T))
    torch.cuda.synchronize()
    lg = lg.cpu().numpy()
    om = O.OracleModel(cfg2, prm2)
    lo, _, _ = om.forward(ids, state=om.new_state(B, eng_cap=T), planes=3, threads=8)
    assert np.max(np.abs(lg - lo)) < 1e-2
    assert np.max(np.abs(lg - lo)) / np.max(np.abs(lo)) < 1e-3
