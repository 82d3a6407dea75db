"""Model files in the reference's naming (ava_amd.checkpoint): a save/load round trip of every
parameter, the recipe read back from an arch string, Ava 0.4's own arch string (release/ava-0.4/
arch.txt, as data) with its optional brain parts reported, and the refusal of a file of another
recipe."""
import os

import numpy as np
import pytest

from ava_amd import checkpoint as ck
from ava_amd import synth

AVA04_ARCH = ("--head-size 64 --timescales fixed --gates channel --value-residual --kwta 1/4 --mlp-act relu2 "
              "--mem-momentum 0.5 --resid-fix --residual dense --lif-init logspaced --lif-scale --spikes int2 --alif "
              "--lif-reset-grad --homeostasis 0.1 --stp --neuromod 3 --dendrite --letters --dopamine --mood --rhythm "
              "--thalamus --cerebellum-head 12288")


@pytest.mark.parametrize("name", ["tiny", "tiny_cb", "small", "tiny_heads"])
def test_round_trip(name, tmp_path):
    cfg = synth.config(name)
    prm = synth.params(cfg, seed=3)
    if cfg.get("cb_units"):
        prm["cb_w"] = np.random.default_rng(4).standard_normal((cfg["cb_units"], cfg["d"])).astype(np.float32)
    path = str(tmp_path / "m.safetensors")
    ck.save_safetensors(path, cfg, prm)
    cfg2, prm2 = ck.load_safetensors(path, ck.arch_of(cfg))
    for k in ("vocab", "d", "layers", "hidden", "kwta_k", "eng_block", "eng_dim", "levels", "alif", "lif_scale",
              "value_residual", "dense", "relu2", "momentum", "head_size", "gate_rank"):
        assert cfg2[k] == cfg[k], k
    assert max(1, cfg2["eng_heads"]) == max(1, cfg.get("eng_heads", 1) or 1)
    assert cfg2.get("cb_units", 0) == cfg.get("cb_units", 0)
    for k in ("tok_emb", "final_norm"):
        assert np.array_equal(prm2[k], prm[k])
    if cfg.get("cb_units"):
        assert np.array_equal(prm2["cb_w"], prm["cb_w"])
    for i, (a, b) in enumerate(zip(prm["blocks"], prm2["blocks"])):
        assert sorted(a) == sorted(b), i
        for f in a:
            if f == "vres" and i == 0:
                assert not b[f].any()  # the first block has no value residual (not stored)
            else:
                assert np.array_equal(a[f], b[f]), (i, f)


def test_ava04_arch_string():
    rec, unsupported = ck.parse_arch(AVA04_ARCH)
    assert rec["alif"] and rec["lif_scale"] and rec["value_residual"] and rec["dense"] and rec["relu2"]
    assert rec["momentum"] == 0.5 and rec["levels"] == 2 and rec["kwta_div"] == 4 and rec["cb_units"] == 12288
    assert unsupported == ["--stp", "--neuromod 3", "--dendrite", "--letters", "--dopamine", "--mood", "--rhythm",
                           "--thalamus"]


def test_unsupported_parts_refused_unless_not_strict(tmp_path):
    cfg = synth.config("tiny")
    path = str(tmp_path / "m.safetensors")
    ck.save_safetensors(path, cfg, synth.params(cfg, seed=1))
    arch = ck.arch_of(cfg) + " --stp --neuromod 3"
    with pytest.raises(ValueError, match="--stp"):
        ck.load_safetensors(path, arch)
    cfg2, _ = ck.load_safetensors(path, arch, strict=False)
    assert cfg2["d"] == cfg["d"]


@pytest.mark.parametrize("arch,msg", [("--gates head --timescales fixed", "channel"),
                                      ("--gates channel --timescales fixed --head-size 32", "64"),
                                      ("--gates channel --timescales fixed --kwta 0.3", "1/n"),
                                      ("--gates channel", "fixed")])
def test_arch_values_this_build_cannot_run(arch, msg):
    with pytest.raises(ValueError, match=msg):
        ck.parse_arch(arch)


@pytest.mark.skipif(not os.path.exists("/root/reference/release/ava-m/model.safetensors"),
                    reason="the reference's release files are not on this machine")
def test_release_file_of_another_recipe_is_refused():
    """release/ava-m is the spiking-only S recipe (b{i}.mem.*, b{i}.mlp.*: no fast-synapse memory):
    read with the safetensors loader, and refused with the reason."""
    with pytest.raises(ValueError, match="fast-synapse memory"):
        ck.load_safetensors("/root/reference/release/ava-m/model.safetensors", "--gates channel --timescales fixed")


def test_engram_heads_default_to_the_reference_geometry(tmp_path):
    """A file with no head count in its metadata (one the reference wrote) reads its engram as heads of
    32 (gpu/model.rs:43 HEAD_SIZE, memory::read): eng.wq [d, d] gives d / 32 heads; an explicit
    override keeps BASELINE's single head of 64."""
    from safetensors.numpy import load_file, save_file
    cfg = synth.config("tiny_heads")
    path = str(tmp_path / "m.safetensors")
    ck.save_safetensors(path, cfg, synth.params(cfg, seed=2))
    bare = str(tmp_path / "bare.safetensors")
    save_file(load_file(path), bare)  # the same tensors, no metadata
    cfg2, _ = ck.load_safetensors(bare, ck.arch_of(cfg))
    assert cfg2["eng_heads"] == cfg["eng_dim"] // 32
    one = synth.config("tiny")
    path1 = str(tmp_path / "one.safetensors")
    ck.save_safetensors(path1, one, synth.params(one, seed=2))
    save_file(load_file(path1), bare)
    assert ck.load_safetensors(bare, ck.arch_of(one))[0]["eng_heads"] == 2  # 64 dims: two heads of 32
    assert ck.load_safetensors(bare, ck.arch_of(one), eng_heads=1)[0]["eng_heads"] == 1
    assert ck.load_safetensors(path1, ck.arch_of(one))[0]["eng_heads"] == 1  # recorded by save


def test_arch_found_beside_the_file(tmp_path):
    """gpu/ckpt.rs:97-112: NAME.arch.txt beside the model file, else arch.txt in its folder; with
    neither the load fails with the names it looked for."""
    cfg = synth.config("tiny")
    prm = synth.params(cfg, seed=5)
    d1 = tmp_path / "own"
    d1.mkdir()
    p1 = str(d1 / "model.safetensors")
    ck.save_safetensors(p1, cfg, prm, write_arch=True)
    assert os.path.isfile(str(d1 / "model.arch.txt"))
    assert ck.load_safetensors(p1)[0]["d"] == cfg["d"]
    d2 = tmp_path / "folder"
    d2.mkdir()
    p2 = str(d2 / "model.safetensors")
    ck.save_safetensors(p2, cfg, prm)
    with pytest.raises(ValueError, match="arch.txt"):
        ck.load_safetensors(p2)
    (d2 / "arch.txt").write_text(ck.arch_of(cfg) + " --stp\n")
    with pytest.raises(ValueError, match="--stp"):
        ck.load_safetensors(p2)  # the folder's options are read (and their optional part refused)
    assert ck.load_safetensors(p2, strict=False)[0]["layers"] == cfg["layers"]
    assert ck.arch_beside(p2)[1] == str(d2 / "arch.txt")
