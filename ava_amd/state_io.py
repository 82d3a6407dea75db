"""Saving and restoring the carried state of B streams, keyed by the model's fingerprint.

Follows the reference's state files (gpu/state.rs:1075-1330): one safetensors file, written through
`path`.tmp and a rename so it is whole or absent (State::save, state.rs:1225-1232), refused on load when
another model wrote it (State::load, state.rs:1236-1246). The fingerprint is FNV-1a 64 over the
configuration text and the same weight samples as Model::fingerprint (state.rs:1075-1092): every 97th
token-embedding value, the whole final norm, every 101st value of each block's MLP down projection, as
little-endian f32. The configuration text is this package's (the reference hashes Rust's Debug print of
its Config), so the two programs' fingerprints differ and neither reads the other's state files.

Tensor names, where the reference has the same quantity (state.rs:1113-1197):
    meta.model [2] u32      the fingerprint, high word first
    meta.blocks [1] u32     the layer count
    meta.seen [B] u32       tokens each stream has consumed
    meta.cap [2] u32        the store's cap and rule: [0, 0] none, [max, 0] oldest first, [max, 1] least read
    eng.reads / eng.age     [B, len] f32 the least-read rule's per-slot read mass and later-query count
    lif.{i}.v / .s / .a     [B, d] membrane, last spikes, adaptation (.a with ALIF)
    mem.{i}.f / .s          [B, nh, hs, hs] the fast weights F and the momentum S (.s with momentum)
    eng.k / eng.v           [B, heads, len, eng_dim / heads] the engram store's filled entries, its dtype
    eng.valid [B] u32       the filled entries of each stream
Names of this package only (the reference keeps the online table on the model, gpu/v51b.rs:189-217,
and its store has no fixed capacity):
    meta.store [2] u32      [capacity, filled] of the engram store
    cb.tab [B, g, d] f32, cb.scale [B] f64, cb.code [B, g] f32   the cerebellum's online table
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np
import torch

FNV_OFFSET = 0xCBF29CE484222325


def fnv1a64(data: bytes, h: int = FNV_OFFSET) -> int:
    """FNV-1a 64 over data, continuing from h (ava_fnv1a64 in the library)."""
    from ._lib import lib
    buf = C.create_string_buffer(bytes(data), len(data))
    return int(lib().ava_fnv1a64(C.cast(buf, C.c_void_p), len(data), C.c_uint64(h)))


# The configuration as hashed: a fixed list of the fields that change the forward or the state's
# layout, each with its default, normalised to int or float (the reference hashes the Debug text of
# its Config, gpu/state.rs:1075-1092, which is likewise one canonical print per configuration).
_CANON = (("vocab", int, None), ("d", int, None), ("layers", int, None), ("hidden", int, None),
          ("kwta_k", int, None), ("head_size", int, 64), ("gate_rank", int, None), ("eng_block", int, -1),
          ("eng_dim", int, 64), ("eng_heads", int, 1), ("eng_half", int, 0), ("levels", int, 2), ("alif", int, 0),
          ("lif_scale", int, 0), ("value_residual", int, 0), ("dense", int, 0), ("relu2", int, 0),
          ("momentum", float, 0.0), ("cap", float, None), ("cb_units", int, 0))
_CANON_CB = (("cb_eta", float, None), ("cb_lr", float, None), ("cb_half", float, 0.0))


def cfg_text(cfg: dict) -> str:
    """The configuration as hashed: the canonical fields in a fixed order, with their defaults filled in
    and their types normalised, so the same model built from arrays or from its file hashes the same.
    The engram's fields count only with an engram, the cerebellum's only with a cerebellum."""
    def val(k, ty, dflt):
        v = cfg.get(k, dflt)
        if v is None:
            return None
        return ty(bool(v)) if ty is int and isinstance(v, bool) else ty(v)

    items = []
    eng = int(cfg.get("eng_block", -1)) >= 0
    for k, ty, dflt in _CANON:
        v = val(k, ty, dflt)
        if k in ("eng_dim", "eng_heads", "eng_half") and not eng:
            continue
        if k == "eng_heads":
            v = max(1, v or 1)
        items.append((k, v))
    if int(cfg.get("cb_units", 0) or 0) > 0:
        items += [(k, val(k, ty, dflt)) for k, ty, dflt in _CANON_CB]
    return repr(items)


def _sample(t, stride: int) -> bytes:
    x = t.detach().reshape(-1)[::stride].to(torch.float32).cpu().numpy() if torch.is_tensor(t) else \
        np.asarray(t, np.float32).reshape(-1)[::stride]
    return np.ascontiguousarray(x, dtype="<f4").tobytes()


def fingerprint(cfg: dict, params: dict) -> int:
    """FNV-1a 64 of the configuration text and weight samples (Model::fingerprint, gpu/state.rs:1075-1092)."""
    h = fnv1a64(cfg_text(cfg).encode())
    h = fnv1a64(_sample(params["tok_emb"], 97), h)
    h = fnv1a64(_sample(params["final_norm"], 1), h)
    for bp in params["blocks"]:
        h = fnv1a64(_sample(bp["w2"], 101), h)
    return h


def _u32(v) -> torch.Tensor:
    return torch.from_numpy(np.array(list(v), dtype=np.uint32))


def _heads(cfg: dict, t: torch.Tensor) -> torch.Tensor:
    """Store rows [B, n, de] as the reference's [B, heads, n, hd] (a view)."""
    nh = max(int(cfg.get("eng_heads", 1) or 1), 1)
    B, n, de = t.shape
    return t.view(B, n, nh, de // nh).permute(0, 2, 1, 3)


def _ints(t: torch.Tensor) -> list:
    if t.dtype != torch.uint32:
        raise ValueError(f"a u32 tensor was expected, not {t.dtype}")
    return [int(x) & 0xFFFFFFFF for x in t.view(torch.int32).tolist()]


def state_tensors(st, cfg: dict, fp: int) -> dict:
    """Every tensor of the state by name, on the host (State::tensors, gpu/state.rs:1113-1223)."""
    L = cfg["layers"]
    n = st.eng_len
    m = {"meta.model": _u32([fp >> 32, fp & 0xFFFFFFFF]), "meta.blocks": _u32([L]),
         "meta.seen": _u32([st.seen] * st.B), "meta.store": _u32([st.eng_cap, n]),
         "meta.cap": _u32([getattr(st, "eng_max", 0), 1 if getattr(st, "eng_rule", "oldest") == "least-read" else 0])}
    cpu = lambda t: t.detach().to("cpu").contiguous()
    for i in range(L):
        m[f"lif.{i}.v"], m[f"lif.{i}.s"] = cpu(st.lif_v[i]), cpu(st.lif_s[i])
        if cfg["alif"]:
            m[f"lif.{i}.a"] = cpu(st.lif_a[i])
        m[f"mem.{i}.f"] = cpu(st.mem_f[i])
        if cfg["momentum"] != 0.0:
            m[f"mem.{i}.s"] = cpu(st.mem_s[i])
    if st.eng_cap:
        m["eng.k"] = cpu(_heads(cfg, st.eng_k[:, :n]))
        m["eng.v"] = cpu(_heads(cfg, st.eng_v[:, :n]))
        m["eng.valid"] = _u32([n] * st.B)
        if getattr(st, "eng_reads", None) is not None:
            m["eng.reads"] = cpu(st.eng_reads[:, :n])
            m["eng.age"] = cpu(st.eng_age[:, :n])
    if st.cb_tab is not None:
        m["cb.tab"], m["cb.scale"], m["cb.code"] = cpu(st.cb_tab), cpu(st.cb_scale), cpu(st.cb_code)
    return m


def save_state(path: str, st, cfg: dict, fp: int) -> None:
    """Write the state to path through path.tmp and a rename (State::save, gpu/state.rs:1225-1232)."""
    from safetensors.torch import save_file
    tmp = os.path.splitext(path)[0] + ".tmp"
    save_file(state_tensors(st, cfg, fp), tmp)
    os.replace(tmp, path)


def load_state(path: str, cfg: dict, fp: int, device="cuda", device_len: bool = False):
    """The state save_state wrote, for the model of fingerprint fp (State::load / State::from_map,
    gpu/state.rs:1236-1330). ValueError when the file holds another model's state or does not fit."""
    import torch
    from safetensors.torch import load_file
    from .model import State
    t = load_file(path)

    def get(k):
        if k not in t:
            raise ValueError(f"{path}: no {k}")
        return t[k]

    have = _ints(get("meta.model"))
    have = (have[0] << 32) | have[1]
    if have != fp:
        raise ValueError(f"{path} was saved by another model (fingerprint {have:016x})")
    nb = _ints(get("meta.blocks"))[0]
    if nb != cfg["layers"]:
        raise ValueError(f"{path}: {nb} blocks, the model has {cfg['layers']}")
    seen = _ints(get("meta.seen"))
    B = len(seen)
    cap, n = _ints(get("meta.store"))
    st = State(cfg, B, cap, device=device, device_len=device_len)
    emax, rule = _ints(get("meta.cap"))
    if rule not in (0, 1):
        raise ValueError(f"{path}: eviction rule {rule} (0 oldest first, 1 least read)")
    st.eng_max = emax
    if rule == 1:
        # counts start at 0 reads and age 0 for a store saved without them (gpu/memory.rs:718)
        st.eng_rule = "least-read"
        st.eng_reads = torch.zeros((B, max(cap, 1)), dtype=torch.float32, device=device)
        st.eng_age = torch.zeros((B, max(cap, 1)), dtype=torch.float32, device=device)

    def put(dst, k):
        src = get(k)
        if tuple(src.shape) != tuple(dst.shape) or src.dtype != dst.dtype:
            raise ValueError(f"{path}: {k} is {tuple(src.shape)} {src.dtype}, the state holds "
                             f"{tuple(dst.shape)} {dst.dtype}")
        dst.copy_(src)

    for i in range(nb):
        put(st.lif_v[i], f"lif.{i}.v")
        put(st.lif_s[i], f"lif.{i}.s")
        if cfg["alif"]:
            put(st.lif_a[i], f"lif.{i}.a")
        put(st.mem_f[i], f"mem.{i}.f")
        if cfg["momentum"] != 0.0:
            put(st.mem_s[i], f"mem.{i}.s")
    if cap:
        if n > cap:
            raise ValueError(f"{path}: {n} stored entries exceed the capacity {cap}")
        put(_heads(cfg, st.eng_k[:, :n]), "eng.k")
        put(_heads(cfg, st.eng_v[:, :n]), "eng.v")
        if _ints(get("eng.valid")) != [n] * B:
            raise ValueError(f"{path}: eng.valid does not match the store length {n}")
        if st.eng_reads is not None and "eng.reads" in t:
            put(st.eng_reads[:, :n], "eng.reads")
            put(st.eng_age[:, :n], "eng.age")
    st.eng_len = n
    if st.eng_len_dev is not None:
        st.eng_len_dev.fill_(n)
    if st.cb_tab is not None:
        put(st.cb_tab, "cb.tab")
        put(st.cb_scale, "cb.scale")
        put(st.cb_code, "cb.code")
    elif "cb.tab" in t:
        raise ValueError(f"{path}: holds a cerebellum table, the model has none")
    if len(set(seen)) != 1:
        raise ValueError(f"{path}: streams of different lengths ({sorted(set(seen))}) are not supported")
    st.seen = seen[0]
    return st
