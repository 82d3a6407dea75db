"""Saved states (ava_amd.state_io) without a GPU: FNV-1a 64 against its published test vectors, the
fingerprint's sampling (gpu/state.rs:1075-1092), and a save/load round trip of every tensor of a
host-side State, with the refusals of State::load (another model's file, another block count)."""
import os

import numpy as np
import pytest
import torch

from ava_amd import state_io as sio
from ava_amd import synth
from ava_amd.model import State


# FNV-1a 64 test vectors from the algorithm's published reference (Fowler, Noll, Vo: "FNV hash", the
# test suite of www.isthe.com/chongo/tech/comp/fnv): the empty string is the offset basis.
@pytest.mark.parametrize("data,want", [(b"", 0xCBF29CE484222325), (b"a", 0xAF63DC4C8601EC8C),
                                       (b"foobar", 0x85944171F73967E8)])
def test_fnv1a64_vectors(data, want):
    assert sio.fnv1a64(data) == want


def test_fnv1a64_continues():
    assert sio.fnv1a64(b"bar", sio.fnv1a64(b"foo")) == sio.fnv1a64(b"foobar")


def test_fingerprint_samples():
    cfg = synth.config("tiny")
    prm = synth.params(cfg, seed=1)
    fp = sio.fingerprint(cfg, prm)
    assert fp == sio.fingerprint(dict(cfg), synth.params(cfg, seed=1))
    # a value the sampling reads (tok_emb every 97th, final_norm all, w2 every 101st) changes it
    for key, idx in (("tok_emb", 97), ("final_norm", 3)):
        p2 = dict(prm)
        t = p2[key].copy()
        t.reshape(-1)[idx] += 1.0
        p2[key] = t
        assert sio.fingerprint(cfg, p2) != fp, key
    b = [dict(x) for x in prm["blocks"]]
    w2 = b[1]["w2"].copy()
    w2.reshape(-1)[202] += 1.0
    b[1]["w2"] = w2
    assert sio.fingerprint(cfg, dict(prm, blocks=b)) != fp
    # one it skips does not
    t = prm["tok_emb"].copy()
    t.reshape(-1)[1] += 1.0
    assert sio.fingerprint(cfg, dict(prm, tok_emb=t)) == fp
    # nor does a torch tensor of the same values
    tp = dict(prm, tok_emb=torch.from_numpy(prm["tok_emb"]))
    assert sio.fingerprint(cfg, tp) == fp
    assert sio.fingerprint(dict(cfg, cap=cfg["cap"] * 2), prm) != fp


def _filled(cfg, B, cap, n, seed):
    st = State(cfg, B, cap, device="cpu")
    g = torch.Generator().manual_seed(seed)
    for t in (st.lif_v, st.lif_s, st.lif_a, st.mem_f, st.mem_s, st.eng_k, st.eng_v, st.cb_tab, st.cb_scale,
              st.cb_code):
        if t is not None:
            t.copy_(torch.randn(t.shape, generator=g, dtype=torch.float64).to(t.dtype))
    st.eng_len, st.seen = n, n
    return st


@pytest.mark.parametrize("name,half", [("tiny", False), ("tiny_cb", False), ("small", True), ("tiny_heads", False)])
def test_round_trip(name, half, tmp_path):
    cfg = dict(synth.config(name), eng_half=half)
    B, cap, n = 3, 40, 17
    st = _filled(cfg, B, cap, n, seed=5)
    fp = 0x0123456789ABCDEF
    path = str(tmp_path / "s.safetensors")
    sio.save_state(path, st, cfg, fp)
    assert os.listdir(tmp_path) == ["s.safetensors"]  # written through .tmp and a rename
    r = sio.load_state(path, cfg, fp, device="cpu")
    assert (r.B, r.eng_cap, r.eng_len, r.seen) == (B, cap, n, n)
    for f in ("lif_v", "lif_s", "lif_a", "mem_f", "mem_s"):
        assert torch.equal(getattr(r, f), getattr(st, f)), f
    assert r.eng_k.dtype == (torch.float16 if half else torch.float32)
    assert torch.equal(r.eng_k[:, :n], st.eng_k[:, :n]) and torch.equal(r.eng_v[:, :n], st.eng_v[:, :n])
    assert not r.eng_k[:, n:].any()  # the unfilled slots are not saved
    if cfg.get("cb_units"):
        for f in ("cb_tab", "cb_scale", "cb_code"):
            assert torch.equal(getattr(r, f), getattr(st, f)), f
    nh = cfg.get("eng_heads", 1)
    ek = sio.state_tensors(st, cfg, fp)["eng.k"]
    assert tuple(ek.shape) == (B, nh, n, cfg["eng_dim"] // nh)  # the reference's [B, heads, S, hd]
    assert torch.equal(ek[:, -1], st.eng_k[:, :n, -(cfg["eng_dim"] // nh):])
    names = set(sio.state_tensors(st, cfg, fp))
    assert {"meta.model", "meta.blocks", "meta.seen", "lif.0.v", "lif.0.s", "lif.0.a", "mem.0.f", "mem.0.s",
            "eng.k", "eng.v", "eng.valid"} <= names


def test_refusals(tmp_path):
    cfg = synth.config("tiny")
    st = _filled(cfg, 2, 8, 5, seed=6)
    path = str(tmp_path / "s.safetensors")
    sio.save_state(path, st, cfg, 7)
    with pytest.raises(ValueError, match="another model"):
        sio.load_state(path, cfg, 8, device="cpu")
    with pytest.raises(ValueError, match="blocks"):
        sio.load_state(path, dict(cfg, layers=3), 7, device="cpu")
    with pytest.raises(ValueError, match="lif.0.v"):
        sio.load_state(path, dict(cfg, d=256, kwta_k=256), 7, device="cpu")
    # no momentum: the S tensors are neither written nor needed
    cfg0 = dict(cfg, momentum=0.0)
    sio.save_state(path, st, cfg0, 7)
    assert "mem.0.s" not in sio.state_tensors(st, cfg0, 7)
    assert not sio.load_state(path, cfg0, 7, device="cpu").mem_s.any()


def test_evict_refuses_a_host_store():
    """The store's cap evicts on the GPU only (ava_engram_evict): a host-side state over its cap is
    refused before anything is launched; under the cap nothing happens."""
    cfg = synth.config("tiny")
    st = _filled(cfg, 2, 20, 13, seed=8)
    st.eng_max = 16
    st.evict()
    assert st.eng_len == 13
    st.eng_max = 5
    with pytest.raises(ValueError):
        st.evict()
    assert st.eng_len == 13


def test_cap_saved_and_refused_rules(tmp_path):
    """meta.cap = [max, rule] (gpu/state.rs:1130, 1262): 0 oldest first, 1 least read with the store's
    counts as eng.reads / eng.age (zeros when a file has none, gpu/memory.rs:718); other rules refused."""
    cfg = synth.config("tiny")
    st = _filled(cfg, 2, 20, 5, seed=9)
    st.eng_max = 12
    path = str(tmp_path / "s.safetensors")
    sio.save_state(path, st, cfg, 3)
    back = sio.load_state(path, cfg, 3, device="cpu")
    assert back.eng_max == 12 and back.eng_rule == "oldest" and back.eng_reads is None
    # least read: the counts travel with the store
    st.eng_rule = "least-read"
    st.eng_reads = torch.rand((2, st.eng_cap), generator=torch.Generator().manual_seed(1))
    st.eng_age = torch.arange(st.eng_cap, dtype=torch.float32).repeat(2, 1)
    sio.save_state(path, st, cfg, 3)
    back = sio.load_state(path, cfg, 3, device="cpu")
    n = st.eng_len
    assert back.eng_rule == "least-read" and back.eng_max == 12
    assert torch.equal(back.eng_reads[:, :n], st.eng_reads[:, :n]) and torch.equal(back.eng_age[:, :n], st.eng_age[:, :n])
    t = sio.state_tensors(st, cfg, 3)
    del t["eng.reads"], t["eng.age"]
    from safetensors.torch import save_file
    save_file(t, path)
    back = sio.load_state(path, cfg, 3, device="cpu")
    assert back.eng_rule == "least-read" and not torch.any(back.eng_reads) and not torch.any(back.eng_age)
    t["meta.cap"] = sio._u32([12, 2])  # no such rule
    save_file(t, path)
    with pytest.raises(ValueError, match="eviction rule"):
        sio.load_state(path, cfg, 3, device="cpu")


@pytest.mark.parametrize("name", ["tiny", "tiny_heads", "tiny_cb"])
def test_array_and_file_models_share_a_fingerprint(name, tmp_path):
    """The same weights built from arrays and read back from their model file key the same states:
    the configuration is hashed in one canonical form (fixed fields, defaults filled, types normalised)."""
    from ava_amd import checkpoint as ck
    cfg = synth.config(name)
    prm = synth.params(cfg, seed=7)
    path = str(tmp_path / "m.safetensors")
    ck.save_safetensors(path, cfg, prm)
    over = dict(cb_eta=cfg["cb_eta"], cb_half=cfg["cb_half"]) if cfg.get("cb_units") else {}
    cfg2, prm2 = ck.load_safetensors(path, ck.arch_of(cfg), **over)
    assert sio.cfg_text(cfg2) == sio.cfg_text(cfg)
    assert sio.fingerprint(cfg2, prm2) == sio.fingerprint(cfg, prm)
    other = dict(cfg, momentum=0.25)
    assert sio.fingerprint(other, prm) != sio.fingerprint(cfg, prm)
