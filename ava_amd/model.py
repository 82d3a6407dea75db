"""The block stack on the HIP path: Model and State with the reference's names (gpu/model.rs,
gpu/state.rs), over ava_model_* of include/ava.h.

    m = Model(cfg, params)              Model::new + set_int8 (model.rs:805, 949-991)
    st = m.state(B, eng_cap)            Model::state (state.rs:593)
    logits = m.forward_with_state(ids, st)   state.rs:684-865 (ids [B, T] int32 on the GPU)
    logits = m.forward(ids)             model.rs:1171: a fresh state per call
    nats = m.cb_learn(logits, next, st) Model::cb_learn (gpu/v51b.rs:600-604, gpu/fast4/cb.rs:25-84)
    m = Model.from_safetensors(path, arch)   a model file in the reference's names (ckpt.rs, model.rs:805-905)
    m.decode_step(ids, st, logits, prev_logits, prev_next)   cb_learn(prev) then forward, overlapped

`params` is a dict of float32 numpy arrays keyed as ava_amd.synth (the reference's VarMap names).
The library raises AvaError on any failure; nothing falls back to another path.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from ._lib import BLOCK_FIELDS, BlockParams, Params, State as _CState, check, config_struct, lib

# The end-of-text id of the reference's byte-pair vocabulary (ava_data::bpe::EOS, data/src/bpe.rs:57),
# at which its generate ends a row (gpu/state.rs:1402, 1436).
EOS = 256


def _ptr(a, keep):
    a = np.ascontiguousarray(a, dtype=np.float32)
    keep.append(a)
    return a.ctypes.data


class State:
    """The carried state of B streams (state.rs:94-116), device tensors. device_len keeps the store
    length on the device too (needed to replay a captured decode step, DecodeGraph)."""

    def __init__(self, cfg: dict, B: int, eng_cap: int = 0, device="cuda", device_len: bool = False):
        L, d, hs, de = cfg["layers"], cfg["d"], cfg["head_size"], cfg["eng_dim"]
        nh = d // hs
        z = lambda *s: torch.zeros(s, dtype=torch.float32, device=device)
        self.B = B
        self.lif_v, self.lif_s, self.lif_a = z(L, B, d), z(L, B, d), z(L, B, d)
        self.mem_f = z(L, B, nh, hs, hs)
        self.mem_s = z(L, B, nh, hs, hs)
        cap = max(eng_cap, 1)
        kv = torch.float16 if cfg.get("eng_half") else torch.float32  # the store's element
        self.eng_k = torch.zeros((B, cap, de), dtype=kv, device=device)
        self.eng_v = torch.zeros((B, cap, de), dtype=kv, device=device)
        self.eng_cap, self.eng_len = eng_cap, 0
        g = cfg.get("cb_units", 0)
        # the cerebellum's online table (CbOnline, gpu/v51b.rs:340-367): delta, scale 1, last code
        self.cb_tab = z(B, g, d) if g else None
        self.cb_scale = torch.ones(B, dtype=torch.float64, device=device) if g else None
        self.cb_code = z(B, g) if g else None
        self.eng_len_dev = torch.zeros(1, dtype=torch.int32, device=device) if device_len else None
        self.seen = 0  # tokens each stream has consumed (State::seen, state.rs:94-116)
        # the store's cap (EngramCap, state.rs:37-69): after a forward the store keeps eng_max entries
        # (0: no cap; the capacity must hold eng_max + T), the last ones (rule "oldest") or those read
        # most per later query ("least-read", which keeps the per-slot counts eng_reads, eng_age)
        self.eng_max = 0
        self.eng_rule = "oldest"
        self.eng_reads = self.eng_age = None

    def select(self, rows) -> "State":
        """A state of the given streams only, in that order (State::select): every tensor's stream axis
        indexed; the store's length, cap and token count are shared."""
        idx = torch.as_tensor(list(rows), dtype=torch.long, device=self.lif_v.device)
        out = object.__new__(State)
        out.__dict__.update(self.__dict__)
        out.B = len(rows)
        for f in ("lif_v", "lif_s", "lif_a", "mem_f", "mem_s"):
            setattr(out, f, getattr(self, f).index_select(1, idx).contiguous())
        for f in ("eng_k", "eng_v", "cb_tab", "cb_scale", "cb_code", "eng_reads", "eng_age"):
            t = getattr(self, f)
            setattr(out, f, t.index_select(0, idx).contiguous() if t is not None else None)
        out.eng_len_dev = self.eng_len_dev.clone() if self.eng_len_dev is not None else None
        return out

    def evict(self):
        """Keep eng_max of the store's entries, in store order (evict, state.rs:518-590), on the device
        (ava_engram_evict: no host round trip). Called by the model after each forward of a capped state.
        "oldest": the last eng_max. "least-read": per stream, the slots rank by (class, value, index) --
        class 1 for a slot some later query could see (age >= 1; value reads / age, its mean mass per later
        query), class 2 for the slots no later query has seen yet -- and the last eng_max of the ranking
        stay."""
        n, mx = self.eng_len, self.eng_max
        # with the length on the device the kernel decides there (a captured step evicts on replay)
        if not mx or (n <= mx and self.eng_len_dev is None):
            return
        if not self.eng_k.is_cuda:
            raise ValueError("evict: the store must be on the GPU (ava_engram_evict runs there)")
        p = lambda t: C.c_void_p(t.data_ptr()) if t is not None else None
        rule = 1 if self.eng_rule == "least-read" else 0
        stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
        check(lib().ava_engram_evict(p(self.eng_k), p(self.eng_v), p(self.eng_reads), p(self.eng_age), self.B,
                                     self.eng_cap, n, p(self.eng_len_dev), self.eng_k.shape[2],
                                     int(self.eng_k.dtype == torch.float16), mx, rule, stream), "ava_engram_evict")
        self.eng_len = min(n, mx)

    def c(self):
        p = lambda t: t.data_ptr() if t is not None else None
        return _CState(lif_v=p(self.lif_v), lif_s=p(self.lif_s), lif_a=p(self.lif_a), mem_f=p(self.mem_f),
                       mem_s=p(self.mem_s), eng_k=p(self.eng_k), eng_v=p(self.eng_v), eng_cap=self.eng_cap,
                       eng_len=self.eng_len, cb_tab=p(self.cb_tab), cb_scale=p(self.cb_scale),
                       cb_code=p(self.cb_code), eng_len_dev=p(self.eng_len_dev), eng_reads=p(self.eng_reads),
                       eng_age=p(self.eng_age))


class Model:
    def __init__(self, cfg: dict, params: dict, planes: int = 3):
        self.cfg = dict(cfg)
        L = cfg["layers"]
        keep = []
        blocks = (BlockParams * L)()
        for i in range(L):
            bp = params["blocks"][i]
            for name in BLOCK_FIELDS:
                if bp.get(name) is not None:
                    setattr(blocks[i], name, _ptr(bp[name], keep))
        prm = Params(tok_emb=_ptr(params["tok_emb"], keep), final_norm=_ptr(params["final_norm"], keep),
                     blocks=C.cast(blocks, C.POINTER(BlockParams)),
                     cb_w=_ptr(params["cb_w"], keep) if params.get("cb_w") is not None else None)
        c = self.cfg
        cb_lr = 0.0
        if c.get("cb_units", 0):
            # the online rate: eta / mean |E_v|^2 (Model::cb_rate, gpu/v51b.rs:606-611) unless given
            from .synth import cb_rate
            cb_lr = c["cb_lr"] if c.get("cb_lr") is not None else cb_rate(params["tok_emb"], c["cb_eta"])
        self.cb_lr = cb_lr
        ccfg = config_struct(c, planes=planes, cb_lr=cb_lr)
        from .state_io import fingerprint
        self.fingerprint = fingerprint(self.cfg, params)  # keys saved states (Model::fingerprint)
        torch.cuda.init()
        h = C.c_void_p()
        check(lib().ava_model_new(C.byref(ccfg), C.byref(prm), C.byref(h)), "ava_model_new")
        self.h = h

    @classmethod
    def from_safetensors(cls, path: str, arch: str | None = None, strict: bool = True, planes: int = 3,
                         **overrides) -> "Model":
        """A model file in the reference's naming (ckpt::load_auto, gpu/ckpt.rs:51-72) with its arch
        string, or with the arch.txt found beside it when arch is None (ava_amd.checkpoint)."""
        from .checkpoint import load_safetensors
        cfg, params = load_safetensors(path, arch, strict=strict, **overrides)
        return cls(cfg, params, planes=planes)

    def __del__(self):
        if getattr(self, "h", None):
            lib().ava_model_free(self.h)
            self.h = None

    def state(self, B: int, eng_cap: int = 0, device_len: bool = False, eng_max: int = 0,
              eng_rule: str = "oldest") -> State:
        """A fresh state of B streams. eng_cap: the store's capacity in entries; eng_max > 0 caps the
        store (EngramCap, state.rs:37-69: eng_cap must hold eng_max + the tokens of the longest
        forward), evicting after each forward by eng_rule, "oldest" or "least-read" (the state then
        keeps per-slot read counts, advanced by each forward)."""
        st = State(self.cfg, B, eng_cap, device_len=device_len)
        if eng_max < 0 or (eng_max and eng_max >= max(eng_cap, 1)):
            raise ValueError(f"eng_max {eng_max}: 0 (no cap) or below the capacity {eng_cap}")
        if eng_rule not in ("oldest", "least-read"):
            raise ValueError(f"engram cap rule {eng_rule!r}: oldest or least-read")
        st.eng_max, st.eng_rule = eng_max, eng_rule
        if eng_rule == "least-read":
            z = lambda: torch.zeros((B, max(eng_cap, 1)), dtype=torch.float32, device=st.lif_v.device)
            st.eng_reads, st.eng_age = z(), z()
        return st

    def save_state(self, st: State, path: str) -> None:
        """Write st to path (safetensors, whole or absent), keyed by this model's fingerprint
        (State::save, gpu/state.rs:1225-1232). Call it between steps: it synchronizes on the copies."""
        from .state_io import save_state
        save_state(path, st, self.cfg, self.fingerprint)

    def load_state(self, path: str, device_len: bool = False) -> State:
        """The state save_state wrote; ValueError when another model wrote it (State::load,
        gpu/state.rs:1236-1246)."""
        from .state_io import load_state
        return load_state(path, self.cfg, self.fingerprint, device="cuda", device_len=device_len)

    def capture_decode(self, st: State, ids: torch.Tensor, logits: torch.Tensor, nxt: torch.Tensor | None = None,
                       nats: torch.Tensor | None = None) -> "DecodeGraph":
        """One decode step (the forward of ids [B, T] into logits, then, with nxt, the online table's
        step) captured as a HIP graph over fixed buffers: fill ids (and nxt) in place, then replay().
        The state needs device_len; call the step eagerly once before capturing (scratch is allocated
        on first use, and a capture must not allocate)."""
        if st.eng_len_dev is None:
            raise ValueError("capture_decode: the state needs device_len=True")
        if st.eng_max and st.eng_rule == "least-read":
            raise ValueError("capture_decode: the least-read counts take the store's length from the host")
        check(lib().ava_model_freeze(self.h, 1), "ava_model_freeze")  # the graph keeps the scratch's addresses
        g = torch.cuda.CUDAGraph()
        n0, s0 = st.eng_len, st.seen
        with torch.cuda.graph(g):
            self.forward_with_state(ids, st, logits)
            if nxt is not None:
                self.cb_learn(logits, nxt, st, nats=nats)
        st.eng_len, st.seen = n0, s0  # the capture ran nothing: the store did not advance
        return DecodeGraph(g, st, ids.shape[1])

    def forward_with_state(self, ids: torch.Tensor, st: State, logits: torch.Tensor | None = None, want_logits=True):
        if not (ids.is_cuda and ids.dtype == torch.int32 and ids.is_contiguous() and ids.dim() == 2):
            raise ValueError("ids: a contiguous [B, T] int32 GPU tensor is required")
        B, T = ids.shape
        self._last_B = 0  # set once the forward is accepted
        if want_logits and logits is None:
            logits = torch.empty((B * T, self.cfg["vocab"]), dtype=torch.float32, device=ids.device)
        cst = st.c()
        stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
        check(lib().ava_model_forward(self.h, C.byref(cst), C.c_void_p(ids.data_ptr()), B, T,
                                      C.c_void_p(logits.data_ptr()) if want_logits else None, stream),
              "ava_model_forward")
        self._last_B = B
        st.eng_len = cst.eng_len
        st.seen += T
        st.evict()
        return logits

    def decode_step(self, ids: torch.Tensor, st: State, logits: torch.Tensor, prev_logits: torch.Tensor | None = None,
                    prev_next: torch.Tensor | None = None, prev_nats: torch.Tensor | None = None):
        """One decode step with the previous token's table step overlapped (ava_model_decode_step): the
        same results as cb_learn(prev_logits, prev_next) then forward_with_state(ids). Alternate two
        logits and two next buffers between steps; prev_* None: no table step (the first token)."""
        if not (ids.is_cuda and ids.dtype == torch.int32 and ids.is_contiguous() and ids.dim() == 2):
            raise ValueError("ids: a contiguous [B, T] int32 GPU tensor is required")
        B, T = ids.shape
        self._last_B = 0  # set once the step is accepted
        V = self.cfg["vocab"]
        if not (logits.is_cuda and logits.dtype == torch.float32 and logits.is_contiguous()
                and logits.numel() >= B * T * V):
            raise ValueError("logits: a contiguous f32 GPU tensor of B*T*vocab entries is required")
        pl = pn = pz = None
        ld = 0
        if prev_logits is not None:
            if prev_next is None or st.cb_tab is None:
                raise ValueError("decode_step: a table step needs prev_next and a state with a table")
            if not (prev_logits.is_cuda and prev_logits.dtype == torch.float32 and prev_logits.dim() == 2
                    and prev_logits.shape[0] == B and prev_logits.stride(1) == 1):
                raise ValueError("prev_logits: [B, vocab] f32 GPU rows with unit column stride are required")
            if prev_logits.data_ptr() == logits.data_ptr():
                raise ValueError("decode_step: logits and prev_logits must be different buffers")
            if not (prev_next.is_cuda and prev_next.dtype == torch.int32 and prev_next.is_contiguous()
                    and prev_next.numel() == B):
                raise ValueError("prev_next: a contiguous [B] int32 GPU tensor is required")
            if prev_nats is not None and not (prev_nats.is_cuda and prev_nats.dtype == torch.float64
                                              and prev_nats.numel() >= B and prev_nats.is_contiguous()):
                raise ValueError("prev_nats: a contiguous f64 GPU tensor of >= B entries is required")
            pl, pn = C.c_void_p(prev_logits.data_ptr()), C.c_void_p(prev_next.data_ptr())
            pz = C.c_void_p(prev_nats.data_ptr()) if prev_nats is not None else None
            ld = prev_logits.stride(0)
        cst = st.c()
        stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
        check(lib().ava_model_decode_step(self.h, C.byref(cst), C.c_void_p(ids.data_ptr()), B, T,
                                          C.c_void_p(logits.data_ptr()), pl, ld, pn, pz, stream),
              "ava_model_decode_step")
        self._last_B = B
        st.eng_len = cst.eng_len
        st.seen += T
        st.evict()
        return logits

    def capture_decode_step(self, st: State, ids: torch.Tensor, logits: torch.Tensor, prev_logits: torch.Tensor,
                            prev_next: torch.Tensor, prev_nats: torch.Tensor | None = None) -> "DecodeGraph":
        """decode_step over fixed buffers as a HIP graph (both streams' work; see capture_decode)."""
        if st.eng_len_dev is None:
            raise ValueError("capture_decode_step: the state needs device_len=True")
        if st.eng_max and st.eng_rule == "least-read":
            raise ValueError("capture_decode_step: the least-read counts take the store's length from the host")
        check(lib().ava_model_freeze(self.h, 1), "ava_model_freeze")
        g = torch.cuda.CUDAGraph()
        n0, s0 = st.eng_len, st.seen
        with torch.cuda.graph(g):
            self.decode_step(ids, st, logits, prev_logits, prev_next, prev_nats)
        st.eng_len, st.seen = n0, s0
        return DecodeGraph(g, st, ids.shape[1])

    def cb_learn(self, logits: torch.Tensor, nxt: torch.Tensor, st: State, nats: torch.Tensor | None = None):
        """One online step of every stream's table (Model::cb_learn): logits [B, >= vocab] f32 GPU rows of
        each stream's last position, nxt [B] int32 GPU (outside [0, vocab): no step). Returns nats [B] f64."""
        if st.cb_tab is None:
            raise ValueError("cb_learn: the state has no cerebellum table (cb_units == 0)")
        B = st.B
        if not (nxt.is_cuda and nxt.dtype == torch.int32 and nxt.is_contiguous() and nxt.numel() == B):
            raise ValueError("nxt: a contiguous [B] int32 GPU tensor is required")
        if not (logits.is_cuda and logits.dtype == torch.float32 and logits.dim() == 2 and logits.shape[0] == B
                and logits.stride(1) == 1):
            raise ValueError("logits: [B, vocab] f32 GPU rows with unit column stride are required")
        if nats is None:
            nats = torch.empty(B, dtype=torch.float64, device=logits.device)
        elif not (nats.is_cuda and nats.dtype == torch.float64 and nats.numel() >= B and nats.is_contiguous()):
            raise ValueError("nats: a contiguous f64 GPU tensor of >= B entries is required")
        cst = st.c()
        stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
        check(lib().ava_model_cb_learn(self.h, C.byref(cst), C.c_void_p(logits.data_ptr()), logits.stride(0),
                                       C.c_void_p(nxt.data_ptr()), B, C.c_void_p(nats.data_ptr()), stream),
              "ava_model_cb_learn")
        return nats

    def generate(self, prompts, max_new: int, pick=None, stop=None, eos: int | None = EOS,
                 batch_rows: int = 256) -> list:
        """Continuations of every prompt with carried state (generate, gpu/state.rs:1392-1458): the
        prompts are read in batched passes, then the rows step together, one token per pass; a row
        leaves at eos (not included; the reference's ava_data::bpe::EOS = 256 by default, as its
        generate always ends a row there; None: rows never stop at a token, as for synthetic
        vocabularies) or when stop(tokens) is true. pick(row, logits [vocab]) chooses
        a token (default: greedy, the lowest id on ties). Rows of one pass share a prompt length
        (this state keeps one store length for all its streams); rows are independent, so the
        grouping does not change any row's tokens. Returns each prompt's tokens."""
        if any(len(p) == 0 for p in prompts):
            raise ValueError("generate: an empty prompt")
        out = [[] for _ in prompts]
        if max_new <= 0:
            return out
        order = sorted(range(len(prompts)), key=lambda r: (len(prompts[r]), r))
        br = max(batch_rows, 1)
        eng = self.cfg["eng_block"] >= 0
        i = 0
        while i < len(order):
            n0 = len(prompts[order[i]])
            group = [r for r in order[i:i + br] if len(prompts[r]) == n0]
            i += len(group)
            st = self.state(len(group), eng_cap=n0 + max_new if eng else 0)
            ids = torch.tensor([prompts[r] for r in group], dtype=torch.int32, device="cuda")
            last = self.forward_with_state(ids, st).view(len(group), n0, -1)[:, -1]
            live = list(group)
            if pick is None and stop is None and eos is None:
                # greedy with nothing that ends a row early: every step's token stays on the device and
                # feeds the next step, so the host reads the tokens once, at the end
                toks = []
                for step in range(max_new):
                    x = torch.argmax(last, dim=1).to(torch.int32).view(-1, 1)
                    toks.append(x)
                    if step + 1 == max_new:
                        break
                    last = self.forward_with_state(x, st)
                got = torch.cat(toks, dim=1).tolist()
                for k, r in enumerate(live):
                    out[r].extend(got[k])
                continue
            for step in range(max_new):
                if pick is None:
                    toks = torch.argmax(last, dim=1).tolist()  # the first (lowest) id of the maximum
                else:
                    toks = [int(pick(r, last[k])) for k, r in enumerate(live)]
                keep, nxt = [], []
                for k, (r, tok) in enumerate(zip(live, toks)):
                    if eos is not None and tok == eos:
                        continue
                    out[r].append(tok)
                    if stop is not None and stop(out[r]):
                        continue
                    keep.append(k)
                    nxt.append(tok)
                if not keep or step + 1 == max_new:
                    break
                if len(keep) != len(live):
                    st = st.select(keep)
                    live = [live[k] for k in keep]
                x = torch.tensor(nxt, dtype=torch.int32, device="cuda").view(-1, 1)
                last = self.forward_with_state(x, st)
        return out

    def forward(self, ids: torch.Tensor):
        B, T = ids.shape
        st = self.state(B, eng_cap=T if self.cfg["eng_block"] >= 0 else 0)
        return self.forward_with_state(ids, st), st

    # the decision trace (ava_model_set_trace)
    def set_trace(self, rows: int | None):
        """Trace the next forwards' discrete decisions into new GPU buffers of `rows` rows (None: off).
        Returns {"spikes": int8 [L, rows, d], "u": f32 [L, rows, hidden], "kth": f32 [L, rows]}; each
        forward fills the next B*T rows (b-major), and trace_rows() tells how many are filled."""
        if rows is None:
            check(lib().ava_model_set_trace(self.h, None, None, None, 0), "ava_model_set_trace")
            self._trace = None
            return None
        c = self.cfg
        L, d, H = c["layers"], c["d"], c["hidden"]
        tr = {"spikes": torch.zeros((L, rows, d), dtype=torch.int8, device="cuda"),
              "u": torch.zeros((L, rows, H), dtype=torch.float32, device="cuda"),
              "kth": torch.zeros((L, rows), dtype=torch.float32, device="cuda")}
        check(lib().ava_model_set_trace(self.h, C.c_void_p(tr["spikes"].data_ptr()), C.c_void_p(tr["u"].data_ptr()),
                                        C.c_void_p(tr["kth"].data_ptr()), rows), "ava_model_set_trace")
        self._trace = tr
        return tr

    def nonfinite(self) -> list:
        """The streams of the last forward whose memory met a non-finite gate, key, query or value (their
        fast weights were left as they were; gpu/model/fstep/arch.rs:780-783's guard). Waits for the
        current stream."""
        n = C.c_int(0)
        stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
        B = getattr(self, "_last_B", 0)
        rows = (C.c_int32 * max(B, 1))()
        check(lib().ava_model_nonfinite(self.h, rows, max(B, 1), C.byref(n), stream), "ava_model_nonfinite")
        return [i for i in range(B) if rows[i]] if n.value else []

    # launch timing by kernel class (ava_model_set_timing / ava_model_timing)
    def set_timing(self, on: bool):
        check(lib().ava_model_set_timing(self.h, int(on)), "ava_model_set_timing")

    def timing(self, reset: bool = False) -> dict:
        cap = 64
        names = (C.c_char_p * cap)()
        calls = (C.c_int * cap)()
        ms = (C.c_double * cap)()
        n = lib().ava_model_timing(self.h, names, calls, ms, cap, int(reset))
        if n < 0:
            raise RuntimeError("ava_model_timing failed: " + lib().ava_last_error().decode())
        return {names[i].decode(): (calls[i], ms[i]) for i in range(min(n, cap))}

    def scratch_bytes(self) -> int:
        return lib().ava_model_scratch_bytes(self.h)


class DecodeGraph:
    """A captured decode step (Model.capture_decode). replay() runs it once on the current stream and
    advances the host's store length as the captured forward advances the device's."""

    def __init__(self, graph, st: State, T: int):
        self.graph, self.st, self.T = graph, st, T

    def replay(self):
        st = self.st
        if st.eng_cap and st.eng_len + self.T > st.eng_cap:
            raise ValueError(f"decode graph: the engram store holds {st.eng_len} of {st.eng_cap} entries")
        self.graph.replay()
        st.eng_len += self.T
        if st.eng_max:
            st.eng_len = min(st.eng_len, st.eng_max)  # the captured eviction ran on the device
        st.seen += self.T
