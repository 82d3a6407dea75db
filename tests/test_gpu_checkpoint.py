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
