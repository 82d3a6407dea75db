"""The float32 training step on the HIP path (ava_train_* of include/ava.h): the loss and every
parameter's gradient of one teacher-forced batch, as the reference's hand-written step computes them
(gpu/model/fwin.rs: loss_and_grads for the Ava-0.4 recipe).

    tr = Trainer(cfg, slope=4.0)             the step for a configuration (ava_amd.synth's keys)
    flat = tr.pack(params)                   the parameters as one flat f32 GPU tensor
    loss, grads = tr.step(flat, ids, targets)   ids, targets [B, T] int32 GPU; grads flat like params
    g = tr.unpack(grads)                     {"tok_emb": ..., "final_norm": ..., "blocks": [{...}]}

The optimizer is the caller's (the reference's AdamW lives outside the step). Nothing falls back to
another path: the library raises AvaError on any failure.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from ._lib import BLOCK_FIELDS, check, config_struct, lib

GLOBAL = ("tok_emb", "final_norm")


class Trainer:
    def __init__(self, cfg: dict, slope: float = 4.0, reset_grad: bool = False):
        self.cfg = dict(cfg)
        torch.cuda.init()
        ccfg = config_struct(self.cfg)
        h = C.c_void_p()
        check(lib().ava_train_new(C.byref(ccfg), float(slope), int(bool(reset_grad)), C.byref(h)), "ava_train_new")
        self.h = h
        self.nparams = lib().ava_train_param_floats(self.h)
        self.slots = {}
        for nm in GLOBAL:
            self.slots[(nm, -1)] = self._slot(nm, -1)
        for i in range(self.cfg["layers"]):
            for nm in BLOCK_FIELDS:
                off, n = self._slot(nm, i)
                if n:
                    self.slots[(nm, i)] = (off, n)
        self.loss = torch.zeros(1, dtype=torch.float32, device="cuda")

    def _slot(self, name, block):
        off, n = C.c_size_t(), C.c_size_t()
        check(lib().ava_train_param_slot(self.h, name.encode(), block, C.byref(off), C.byref(n)), "ava_train_param_slot")
        return off.value, n.value

    def __del__(self):
        if getattr(self, "h", None):
            lib().ava_train_free(self.h)
            self.h = None

    def pack(self, params: dict) -> torch.Tensor:
        """The flat f32 GPU parameter buffer from ava_amd.synth-style numpy (or torch) arrays."""
        flat = np.zeros(self.nparams, np.float32)
        for (nm, i), (off, n) in self.slots.items():
            src = params[nm] if i < 0 else params["blocks"][i].get(nm)
            if src is None:
                raise ValueError(f"pack: block {i} has no {nm}")
            a = np.asarray(src.cpu() if isinstance(src, torch.Tensor) else src, np.float32).reshape(-1)
            if a.size != n:
                raise ValueError(f"pack: {nm} of block {i} has {a.size} values, {n} expected")
            flat[off:off + n] = a
        return torch.from_numpy(flat).cuda()

    def unpack(self, flat: torch.Tensor) -> dict:
        """Views of a flat buffer in the parameters' shapes (the blocks' matrices as [din, dout])."""
        c = self.cfg
        out = {"blocks": [dict() for _ in range(c["layers"])]}
        for (nm, i), (off, n) in self.slots.items():
            v = flat[off:off + n]
            shape = _shape(c, nm, i)
            (out if i < 0 else out["blocks"][i])[nm] = v.view(shape)
        return out

    def step(self, flat: torch.Tensor, ids: torch.Tensor, targets: torch.Tensor, grads: torch.Tensor | None = None):
        """Loss (a 1-element GPU tensor) and the flat gradient buffer of one batch."""
        for t, nm in ((ids, "ids"), (targets, "targets")):
            if not (t.is_cuda and t.dtype == torch.int32 and t.is_contiguous() and t.dim() == 2):
                raise ValueError(f"{nm}: a contiguous [B, T] int32 GPU tensor is required")
        if targets.shape != ids.shape:
            raise ValueError("targets: the shape of ids is required")
        if not (flat.is_cuda and flat.dtype == torch.float32 and flat.numel() == self.nparams and flat.is_contiguous()):
            raise ValueError("params: the flat f32 GPU buffer of pack() is required")
        if grads is None:
            grads = torch.empty_like(flat)
        B, T = ids.shape
        stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
        check(lib().ava_train_step(self.h, C.c_void_p(flat.data_ptr()), C.c_void_p(ids.data_ptr()),
                                   C.c_void_p(targets.data_ptr()), B, T, C.c_void_p(grads.data_ptr()),
                                   C.c_void_p(self.loss.data_ptr()), stream), "ava_train_step")
        return self.loss, grads

    def decisions(self, B: int, T: int) -> dict:
        """The last step's spikes [L, B*T, d] int8, wide-layer u [L, B*T, hidden] and k-th values [L, B*T]."""
        c = self.cfg
        L, N = c["layers"], B * T
        spk = torch.empty((L, N, c["d"]), dtype=torch.int8, device="cuda")
        u = torch.empty((L, N, c["hidden"]), dtype=torch.float32, device="cuda")
        kth = torch.empty((L, N), dtype=torch.float32, device="cuda")
        stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
        check(lib().ava_train_decisions(self.h, C.c_void_p(spk.data_ptr()), C.c_void_p(u.data_ptr()),
                                        C.c_void_p(kth.data_ptr()), stream), "ava_train_decisions")
        return {"spikes": spk, "u": u, "kth": kth}


def _shape(c, nm, i):
    d, H, V, r, de = c["d"], c["hidden"], c["vocab"], c["gate_rank"], c["eng_dim"]
    nh = d // c["head_size"]
    return {
        "tok_emb": (V, d), "win": (d, d), "wout": (d, d), "wq": (d, d), "wk": (d, d), "wv": (d, d), "we": (d, d),
        "wg": (d, d), "wo": (d, d), "wa": (d, nh), "wb": (d, nh), "ba": (nh,), "bb": (nh,), "wa1": (d, r),
        "wb1": (d, r), "wa2": (r, d), "wb2": (r, d), "vres": (2,), "ewq": (d, de), "ewk": (d, de), "ewv": (d, de),
        "ewo": (de, d), "w1": (d, H), "w2": (H, d), "dense": (i + 2,),
    }.get(nm, (d,))
