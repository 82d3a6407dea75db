"""Model files in the reference's naming: safetensors in and out, and the block recipe from an arch
string (release/ava-0.4/arch.txt).

Names (gpu/src/model.rs:805-905, gpu/src/arch.rs:806-860, gpu/src/v51b.rs:291): `tok_emb`,
`final.norm`, `cbh.wo`; per block i the spiking layer `b{i}.mem.{norm,win,beta,wout}` (+ `theta`
with --homeostasis, `arho` / `again` with --alif), the fast-synapse memory `b{i}.hebb.{norm,wq,wk,
wv,wo,wg,wa,ba,wb,bb}` with the channel gates' `wa1,wa2,wb1,wb2,we` and (i > 0) `vres`, the sparse
MLP `b{i}.mlp.{norm,w1,w2}`, the dense residual `b{i}.dense`, and the engram read `b{i}.eng.{norm,
wq,wk,wv,wo}`. The gate offsets (`off`) are not stored: they follow from the head count
(Timescales::Fixed, gpu/arch.rs:656-666). Files are read with the safetensors numpy loader (no code
runs from the file).

The arch flags this build runs (gpu/arch.rs:270-405): --head-size 64, --timescales fixed, --gates
channel, --kwta 1/n, --mlp-act relu|relu2, --mem-momentum, --residual plain|dense, --spikes
ternary|int2, --alif, --lif-scale, --value-residual, --gate silu, --gate-rank <= 32 and
--cerebellum-head G; flags that only change training or initialisation (--lif-init,
--surrogate-slope, --lif-reset-grad, --resid-fix, --homeostasis) are accepted. Every other flag (the
optional brain parts) is reported: load_safetensors refuses them unless strict=False, in which case
those parts are left out of the forward.
"""
from __future__ import annotations

import os

import numpy as np

from . import synth

BLOCK_NAMES = {
    "lif_norm": "b{i}.mem.norm", "win": "b{i}.mem.win", "beta_p": "b{i}.mem.beta", "wout": "b{i}.mem.wout",
    "theta": "b{i}.mem.theta", "arho": "b{i}.mem.arho", "again": "b{i}.mem.again",
    "mem_norm": "b{i}.hebb.norm", "wq": "b{i}.hebb.wq", "wk": "b{i}.hebb.wk", "wv": "b{i}.hebb.wv",
    "wo": "b{i}.hebb.wo", "wg": "b{i}.hebb.wg", "wa": "b{i}.hebb.wa", "ba": "b{i}.hebb.ba", "wb": "b{i}.hebb.wb",
    "bb": "b{i}.hebb.bb", "we": "b{i}.hebb.we", "wa1": "b{i}.hebb.wa1", "wa2": "b{i}.hebb.wa2",
    "wb1": "b{i}.hebb.wb1", "wb2": "b{i}.hebb.wb2", "vres": "b{i}.hebb.vres",
    "mlp_norm": "b{i}.mlp.norm", "w1": "b{i}.mlp.w1", "w2": "b{i}.mlp.w2", "dense": "b{i}.dense",
    "eng_norm": "b{i}.eng.norm", "ewq": "b{i}.eng.wq", "ewk": "b{i}.eng.wk", "ewv": "b{i}.eng.wv",
    "ewo": "b{i}.eng.wo",
}
TOP_NAMES = {"tok_emb": "tok_emb", "final_norm": "final.norm", "cb_w": "cbh.wo"}
ENGRAM = ("eng_norm", "ewq", "ewk", "ewv", "ewo")
LIF_THRESHOLD = 1.0  # gpu/arch.rs: the base threshold without --homeostasis

# flags with no effect on the forward of a trained model
_TRAINING_ONLY = {"--lif-init": 1, "--surrogate-slope": 1, "--lif-reset-grad": 0, "--resid-fix": 0,
                  "--homeostasis": 1}


def parse_arch(text: str):
    """The recipe of an arch string: (settings for synth-style configs, unsupported flags). Raises
    ValueError on values this build cannot run (gpu/arch.rs:270-405 for the flags' meanings)."""
    toks = text.split()
    cfg, unsupported = {}, []
    defaults = dict(levels=2, alif=False, lif_scale=False, value_residual=False, dense=False, relu2=False,
                    momentum=0.0, head_size=64, gate_rank=synth.GATE_RANK, kwta_div=1)
    cfg.update(defaults)
    seen_gates = seen_ts = False
    i = 0
    while i < len(toks):
        key = toks[i]
        val = toks[i + 1] if i + 1 < len(toks) else None
        take = 1
        if key == "--value-residual":
            cfg["value_residual"] = True
        elif key == "--lif-scale":
            cfg["lif_scale"] = True
        elif key == "--alif":
            cfg["alif"] = True
        elif key in _TRAINING_ONLY:
            take = 1 + _TRAINING_ONLY[key]
        elif key in ("--head-size", "--timescales", "--gates", "--kwta", "--mlp-act", "--mem-momentum", "--residual",
                     "--spikes", "--gate", "--gate-rank", "--cerebellum-head"):
            if val is None:
                raise ValueError(f"{key} needs a value")
            take = 2
            if key == "--head-size":
                if int(val) != 64:
                    raise ValueError(f"--head-size {val}: this build runs 64")
                cfg["head_size"] = 64
            elif key == "--timescales":
                if val != "fixed":
                    raise ValueError(f"--timescales {val}: this build runs fixed")
                seen_ts = True
            elif key == "--gates":
                if val != "channel":
                    raise ValueError(f"--gates {val}: this build runs channel")
                seen_gates = True
            elif key == "--kwta":
                a, _, b = val.partition("/")
                f = float(a) / float(b) if b else float(a)
                div = round(1.0 / f)
                if not (0.0 < f <= 1.0) or abs(1.0 / div - f) > 1e-9:
                    raise ValueError(f"--kwta {val}: a fraction 1/n")
                cfg["kwta_div"] = div
            elif key == "--mlp-act":
                if val not in ("relu", "relu2"):
                    raise ValueError(f"--mlp-act {val}: relu or relu2")
                cfg["relu2"] = val == "relu2"
            elif key == "--mem-momentum":
                cfg["momentum"] = float(val)
            elif key == "--residual":
                if val not in ("plain", "dense"):
                    raise ValueError(f"--residual {val}: plain or dense")
                cfg["dense"] = val == "dense"
            elif key == "--spikes":
                if val not in ("ternary", "int2"):
                    raise ValueError(f"--spikes {val}: ternary or int2")
                cfg["levels"] = 2 if val == "int2" else 1
            elif key == "--gate":
                if val != "silu":
                    raise ValueError(f"--gate {val}: this build runs silu")
            elif key == "--gate-rank":
                if not 0 < int(val) <= 32:
                    raise ValueError(f"--gate-rank {val}: 1..32")
                cfg["gate_rank"] = int(val)
            elif key == "--cerebellum-head":
                cfg["cb_units"] = int(val)
        elif key.startswith("--"):
            take = 2 if val is not None and not val.startswith("--") else 1
            unsupported.append(" ".join(toks[i:i + take]))
        else:
            raise ValueError(f"arch: unexpected token {key!r}")
        i += take
    if not (seen_gates and seen_ts):
        raise ValueError("arch: this build runs the per-channel gates with fixed timescales "
                         "(--gates channel --timescales fixed)")
    return cfg, unsupported


# The engram's head size in the reference (gpu/model.rs:43 HEAD_SIZE, read by memory::read,
# gpu/memory.rs:610-700). A file this package writes records its own head count in the safetensors
# metadata under this key (BASELINE's single head of 64 is not the reference's geometry).
ENGRAM_HEAD = 32
META_ENG_HEADS = "ava.eng_heads"


def _tensors(path):
    from safetensors.numpy import load_file
    return load_file(path)


def _metadata(path):
    from safetensors import safe_open
    with safe_open(path, framework="np") as f:
        return f.metadata() or {}


def arch_name(path: str) -> str:
    """NAME.arch.txt for the model file NAME.safetensors (gpu/ckpt.rs:92-95: the last extension
    replaced by arch.txt)."""
    root, ext = os.path.splitext(path)
    return (root if ext else path) + ".arch.txt"


def arch_beside(path: str):
    """The block options a model file was made with and the file they came from (gpu/ckpt.rs:97-112):
    NAME.arch.txt beside the model file, else arch.txt in its folder; None when neither exists."""
    for p in (arch_name(path), os.path.join(os.path.dirname(os.path.abspath(path)), "arch.txt")):
        if os.path.isfile(p):
            with open(p) as f:
                return f.read().strip(), p
    return None


def write_arch_beside(path: str, cfg: dict) -> str:
    """Write cfg's block options as NAME.arch.txt beside the model file (gpu/ckpt.rs:114-124), so the
    file loads without an arch argument. Returns the path written."""
    p = arch_name(path)
    with open(p, "w") as f:
        f.write(arch_of(cfg) + "\n")
    return p


def load_safetensors(path: str, arch: str | None = None, strict: bool = True, **overrides):
    """(cfg, params) of a model file in the reference's naming. The block options come from `arch`, or
    when it is None from the arch.txt found beside the file (arch_beside; ValueError if there is none:
    this build runs only models with block options). Dimensions come from the tensors (d and vocab from
    tok_emb, layers from b{i}.mem.win, hidden from b0.mlp.w1, the engram block and width from
    b{i}.eng.wq); the engram's heads are the reference's heads of 32 (eng_dim / 32) unless the file's
    metadata records another count. overrides set the rest (cap, cb_eta, cb_half, eng_half,
    eng_heads)."""
    if arch is None:
        found = arch_beside(path)
        if found is None:
            raise ValueError(f"{path}: no block options given and none beside the file "
                             f"({arch_name(path)} or arch.txt in its folder)")
        arch = found[0]
    rec, unsupported = parse_arch(arch)
    if unsupported and strict:
        raise ValueError("arch: parts this build does not run: " + ", ".join(unsupported))
    t = _tensors(path)
    if "tok_emb" not in t:
        raise ValueError(f"{path}: no tok_emb")
    V, d = t["tok_emb"].shape
    layers = 0
    while f"b{layers}.mem.win" in t:
        layers += 1
    if layers == 0 or "b0.hebb.wq" not in t:
        raise ValueError(f"{path}: not a model with the spiking layer and fast-synapse memory per block "
                         f"(b{{i}}.mem.win, b{{i}}.hebb.wq)")
    hidden = t["b0.mlp.w1"].shape[1]
    eng = [i for i in range(layers) if f"b{i}.eng.wq" in t]
    if len(eng) > 1:
        raise ValueError(f"{path}: engram reads in blocks {eng} (this build runs one)")
    eng_block = eng[0] if eng else -1
    eng_dim = t[f"b{eng_block}.eng.wq"].shape[1] if eng else 64
    meta = _metadata(path)
    eng_heads = int(meta[META_ENG_HEADS]) if META_ENG_HEADS in meta else max(1, eng_dim // ENGRAM_HEAD)
    cfg = dict(vocab=V, d=d, layers=layers, hidden=hidden, kwta_k=hidden // rec.pop("kwta_div"),
               eng_block=eng_block, eng_dim=eng_dim, eng_heads=eng_heads if eng else 1, cap=synth.MEM_CAP,
               cb_units=rec.pop("cb_units", 0))
    cfg.update(rec)
    if cfg["cb_units"]:
        cfg.update(cb_eta=0.3, cb_half=256.0)
    cfg.update(overrides)
    nh = d // cfg["head_size"]
    off = np.repeat(synth.logit(synth.gate_gammas(nh)), cfg["head_size"]).astype(np.float32)
    blocks = []
    for i in range(layers):
        b = {}
        for f, pat in BLOCK_NAMES.items():
            name = pat.format(i=i)
            if f in ENGRAM and i != eng_block:
                continue
            if name in t:
                b[f] = np.ascontiguousarray(t[name], dtype=np.float32)
            elif f == "theta":
                b[f] = np.full(d, LIF_THRESHOLD, np.float32)
            elif f == "vres" and (i == 0 or not cfg["value_residual"]):
                b[f] = np.zeros(2, np.float32)
            elif f in ("arho", "again") and not cfg["alif"]:
                b[f] = np.zeros(d, np.float32)
            elif f == "dense" and not cfg["dense"]:
                b[f] = np.zeros(i + 2, np.float32)
            else:
                raise ValueError(f"{path}: {name} is missing")
        b["off"] = off
        blocks.append(b)
    params = {"tok_emb": np.ascontiguousarray(t["tok_emb"], dtype=np.float32),
              "final_norm": np.ascontiguousarray(t["final.norm"], dtype=np.float32), "blocks": blocks}
    if "cbh.wo" in t:
        params["cb_w"] = np.ascontiguousarray(t["cbh.wo"], dtype=np.float32)
    return cfg, params


def save_safetensors(path: str, cfg: dict, params: dict, write_arch: bool = False):
    """Write params in the reference's naming (the inverse of load_safetensors: `off` is not stored,
    `vres` only for blocks after the first, the engram only in its block). The engram's head count goes
    into the file's metadata. With write_arch, NAME.arch.txt is written beside it (write_arch_beside)."""
    from safetensors.numpy import save_file
    out = {TOP_NAMES[k]: np.ascontiguousarray(params[k], dtype=np.float32) for k in ("tok_emb", "final_norm")}
    if params.get("cb_w") is not None:
        out["cbh.wo"] = np.ascontiguousarray(params["cb_w"], dtype=np.float32)
    for i, b in enumerate(params["blocks"]):
        for f, pat in BLOCK_NAMES.items():
            if f not in b or (f == "vres" and i == 0) or (f in ENGRAM and i != cfg["eng_block"]):
                continue
            out[pat.format(i=i)] = np.ascontiguousarray(b[f], dtype=np.float32)
    meta = {}
    if cfg.get("eng_block", -1) >= 0:
        meta[META_ENG_HEADS] = str(max(1, int(cfg.get("eng_heads", 1) or 1)))
    save_file(out, path, metadata=meta or None)
    if write_arch:
        write_arch_beside(path, cfg)


def arch_of(cfg: dict) -> str:
    """The arch string of a configuration (the flags parse_arch reads back)."""
    f = ["--head-size 64", "--timescales fixed", "--gates channel", f"--kwta 1/{cfg['hidden'] // cfg['kwta_k']}",
         "--mlp-act " + ("relu2" if cfg["relu2"] else "relu"), f"--mem-momentum {cfg['momentum']}",
         "--residual " + ("dense" if cfg["dense"] else "plain"), "--spikes " + ("int2" if cfg["levels"] == 2 else "ternary"),
         f"--gate-rank {cfg['gate_rank']}"]
    f += [flag for flag, on in (("--alif", cfg["alif"]), ("--lif-scale", cfg["lif_scale"]),
                                ("--value-residual", cfg["value_residual"])) if on]
    if cfg.get("cb_units"):
        f.append(f"--cerebellum-head {cfg['cb_units']}")
    return " ".join(f)
