"""BASELINE.json's standalone configs at their full workloads, through the C ABI, against the oracle.

config[1]: the LIF scan at B=64, T=2048, C=2048 on the kernel the library picks for that size (the
one bench.py times): spikes, v_T, a_T and theta_T bit for bit (gpu/lif_gen.rs:379-453 asserts exact
spikes and state).
config[2]: the plain delta rule at B=32, H=8, T=4096, d=64 in chunks of 64 against the f64
recurrence (gpu/mem_gen.rs:220-273 with alpha = 1, e = k, one beta per head, no momentum): read-outs
and final state within 1e-4 relative of the largest magnitude (north_star's fp32-state bar; the
chunked form against the recurrence is pinned to 1e-4 by gpu/arch/tests.rs:704-750).
config[3]: the d=1024 8-block stack at B=2, T=2048 (config[3]'s model and sequence length on two of its
64 streams) against the oracle's forward with the GPU's decisions forced (tests/forced.py).
config[0]: the d=512 model, a 512-token prompt and 128 greedy steps (B=1), the same bars.
config[4]: 256 streams prefilled with 32,768 random tokens on the GPU, then 8 decode steps with the
online table step; two streams' state is copied into the oracle, which steps them with the GPU's
decisions forced (the bars of tests/test_gpu_cb.py for the table).
"""
import forced as F
import numpy as np
import pytest
import torch

from ava_amd import synth
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def cuda(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def rel(a, b):
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def sig(x):
    return (1.0 / (np.exp(-np.asarray(x, np.float32)) + np.float32(1.0))).astype(np.float32)


def test_config1_lif_full_size_bit_exact(dev):
    """config[1] in full: cur ~N(0,1) [64, 2048, 2048]; beta = sigmoid(U(1.5, 4.5)); theta 1, ALIF
    rho 0.95 and gain 0.05; int2 spikes with subtract reset."""
    from ava_amd import ops
    B, T, D = 64, 2048, 2048
    rng = np.random.default_rng(101)
    cur = rng.standard_normal((B, T, D), dtype=np.float32)
    beta = sig(rng.uniform(1.5, 4.5, D))
    ps = np.concatenate([beta, np.ones(D, np.float32), np.full(D, 0.95, np.float32),
                         np.full(D, 0.05, np.float32)]).astype(np.float32)
    print(f"config[1] LIF B={B} T={T} D={D}: GPU scan", flush=True)
    spk, st, th = ops.lif_gen(cuda(cur), cuda(beta), cuda(ps[D:2 * D]), (cuda(ps[2 * D:3 * D]), cuda(ps[3 * D:])),
                              levels=2, signed=True, th_out=True)
    spk_g, v_g, a_g, th_g = host(spk), host(st.v), host(st.a), host(th)
    del spk, st, th
    print("config[1] LIF: oracle scan", flush=True)
    spk_o, v_o, s_o, a_o = O.lif_scan(cur, ps, levels=2, signed=True, alif=True)
    assert np.array_equal(spk_g, spk_o)
    assert np.array_equal(v_g.view(np.uint32), v_o.view(np.uint32))
    assert np.array_equal(a_g.view(np.uint32), a_o.view(np.uint32))
    th_o = (ps[D:2 * D][None, :] + a_o * ps[3 * D:][None, :]).astype(np.float32)
    assert np.array_equal(th_g.view(np.uint32), th_o.view(np.uint32))
    counts = np.bincount((spk_o.reshape(-1).astype(np.int16) + 2), minlength=5)
    print("spike counts -2..2:", counts.tolist(), flush=True)
    assert counts[0] > 0 and counts[4] > 0  # both levels occur on both sides


def test_config2_delta_rule_full_size(dev):
    """config[2] in full: q, k L2-normalised N(0,1); v N(0,1); beta = sigmoid(N(0,1)) per token and
    head; W_0 = 0; chunks of 64."""
    from ava_amd import ops
    Bn, H, T, hs = 32, 8, 4096, 64
    BH = Bn * H
    rng = np.random.default_rng(202)
    q = rng.standard_normal((BH, T, hs), dtype=np.float32)
    k = rng.standard_normal((BH, T, hs), dtype=np.float32)
    q /= np.linalg.norm(q, axis=2, keepdims=True)
    k /= np.linalg.norm(k, axis=2, keepdims=True)
    v = rng.standard_normal((BH, T, hs), dtype=np.float32)
    beta = sig(rng.standard_normal((BH, T)))
    print(f"config[2] delta rule BH={BH} T={T}: GPU chunked form", flush=True)
    y, Fw = ops.delta_rule_from(cuda(q), cuda(k), cuda(v), cuda(beta))
    y, Fw = host(y), host(Fw)
    print("config[2] delta rule: oracle f64 recurrence", flush=True)
    la = np.zeros((BH, T, 1), np.float32)
    y64, F64, _ = O.mem_rec_f64(q, k, k, v, la, beta[:, :, None])
    ry, rF = rel(y, y64), rel(Fw, F64)
    print(f"rel y {ry:.2e}  rel F {rF:.2e}", flush=True)
    assert ry < 1e-4 and rF < 1e-4


@pytest.mark.parametrize("seed", [41, 47])
def test_config3_stack_full_length(seed, dev):
    """config[3]'s model (d 1024, 8 blocks, wide 4096 / k 1024, 16 heads, engram in block 4, vocab
    8192) over 2 streams of config[3]'s 2048 tokens: logits within 1e-2 on every row, every spike and
    kWTA decision, membranes within 1e-4 of the oracle. The fast weights are measured against the same
    forced forward in float64 (oracle/forward64.py): the GPU's distance from it, summed over blocks and
    at its largest block, within 1.5x the f32 oracle's own (tests/forced.py, check_state)."""
    F.run_forced("ava04_d1024", 2, 2048, seed=seed, f64=True)


def test_config3_rows_split_across_forwards_give_the_same_bits(dev):
    """config[3]'s model over 32 streams of 2048 tokens (65,536 rows: the memory norm and its gate
    projections in one launch, rms_gate_many) equals the same streams run as two forwards of 16 (32,768
    rows: rms_planes then gate_gemm, no fused launch) bit for bit: logits and every carried state. Every
    kernel of the stack computes a row (or a stream) the same way at any row count, so any difference
    is a fused-path defect; the oracle pins the two-launch path (test_config3_stack_full_length)."""
    from ava_amd.model import Model
    cfg = synth.config("ava04_d1024")
    m = Model(cfg, synth.params(cfg, seed=43))
    B, T = 32, 2048
    ids = torch.from_numpy(np.random.default_rng(44).integers(0, cfg["vocab"], (B, T)).astype(np.int32)).cuda()
    print(f"config[3] rows split B={B} T={T}", flush=True)
    st = m.state(B, eng_cap=T)
    whole = m.forward_with_state(ids, st)
    halves, sts = [], []
    for h in range(2):
        sh = m.state(B // 2, eng_cap=T)
        halves.append(m.forward_with_state(ids[h * B // 2:(h + 1) * B // 2].contiguous(), sh))
        sts.append(sh)
    torch.cuda.synchronize()
    assert torch.equal(whole, torch.cat(halves, dim=0))
    for name in ("lif_v", "lif_s", "lif_a", "mem_f", "mem_s"):
        full = getattr(st, name)
        parts = [getattr(x, name) for x in sts]
        # state tensors are [L][B][...]: the stream axis is 1
        assert torch.equal(full, torch.cat(parts, dim=1)), name
    for name in ("eng_k", "eng_v"):  # [B][cap][de]
        assert torch.equal(getattr(st, name), torch.cat([getattr(x, name) for x in sts], dim=0)), name


def test_config0_greedy_512_prompt_128_steps(dev):
    """config[0]: the d=512 model, one stream, a 512-token prompt and 128 greedy steps (argmax, the
    lowest id on ties) as Model.generate runs them (one forward per token with carried state). The
    oracle reads the prompt and the GPU's 127 fed-back tokens teacher-forced with the GPU's decisions
    forced; every row's logits are within 1e-2, so each GPU pick is within 2e-2 of the oracle's best."""
    from ava_amd.model import Model
    cfg = synth.config("ava04_d512")
    prm = synth.params(cfg, seed=51)
    P, NEW = 512, 128
    prompt = np.random.default_rng(52).integers(0, cfg["vocab"], P).astype(np.int32)
    print(f"config[0] greedy prompt={P} new={NEW}", flush=True)
    m = Model(cfg, prm)
    st = m.state(1, eng_cap=P + NEW)
    tr = m.set_trace(P + NEW - 1)
    lgs = [F.host(m.forward_with_state(torch.from_numpy(prompt[None]).cuda(), st))]
    toks = []
    for step in range(NEW):
        tok = int(np.argmax(lgs[-1][-1]))
        toks.append(tok)
        if step + 1 == NEW:
            break
        lgs.append(F.host(m.forward_with_state(torch.tensor([[tok]], dtype=torch.int32, device="cuda"), st)))
    lg = np.concatenate(lgs, axis=0)
    dec = F.gpu_decisions(tr, np.arange(P + NEW - 1))
    m.set_trace(None)
    assert Model(cfg, prm).generate([prompt.tolist()], NEW, eos=None)[0] == toks  # generate's own loop
    seq = np.concatenate([prompt, np.asarray(toks[:-1], np.int32)])[None]
    om = O.OracleModel(cfg, prm)
    lo, so, otr = F.forced_oracle(om, seq, dec, om.new_state(1, eng_cap=P + NEW))
    err = float(np.max(np.abs(lg - lo)))
    print(f"config[0]: logits max abs err {err:.2e} over {lg.shape[0]} rows", flush=True)
    assert err < 1e-2
    F.check_state(so, st)
    F.check_decisions(cfg, dec, otr, "config[0]")
    rows = lo[P - 1:]
    picked = rows[np.arange(NEW), toks]
    assert np.all(picked >= rows.max(axis=1) - 2e-2)
    agree = np.mean(np.argmax(rows, axis=1) == np.asarray(toks))
    print(f"config[0]: oracle argmax agrees on {agree:.3f} of the steps", flush=True)


def test_config4_decode_after_32768_token_prefill(dev):
    """config[4]: 256 streams, each prefilled with 32,768 random tokens (fp16 engram store, the
    12,288-unit online table with a 256-token half-life), then 8 steps of one token per stream, each
    followed by the table's learning step on the next token. Streams 0 and 173 are copied into the
    oracle after the prefill and stepped there with the GPU's decisions forced: logits within 1e-2,
    nats and the final tables within 1e-4 relative, codes within 1e-5, the carried state within the
    state bars."""
    from ava_amd.model import Model
    cfg = synth.config("ava04_d1024_decode")
    prm = synth.params(cfg, seed=61)
    B, PRE, STEPS, PIECE = 256, 32768, 8, 512
    V = cfg["vocab"]
    sel = [0, 173]
    m = Model(cfg, prm)
    st = m.state(B, eng_cap=PRE + STEPS)
    g = torch.Generator(device="cuda").manual_seed(62)
    print(f"config[4] prefill {B} streams x {PRE} tokens", flush=True)
    for done in range(0, PRE, PIECE):
        ids = torch.randint(0, V, (B, PIECE), device="cuda", generator=g, dtype=torch.int32)
        m.forward_with_state(ids, st, want_logits=False)
        if done % 8192 == 0:
            print(f"config[4] prefill {done + PIECE} tokens", flush=True)
    torch.cuda.synchronize()
    # the two streams' state, as the oracle holds it (the fp16 store's values exactly as f32)
    sub = st.select(sel)
    om = O.OracleModel(cfg, prm)
    so = om.new_state(len(sel), eng_cap=PRE + STEPS)
    for k in ("lif_v", "lif_s", "lif_a", "mem_f", "mem_s"):
        so[k][...] = F.host(getattr(sub, k))
    for k in ("eng_k", "eng_v"):
        so[k][:, :PRE] = F.host(getattr(sub, k)[:, :PRE].float())
    so["eng_len"] = PRE
    so["cb_tab"][...] = F.host(sub.cb_tab)
    so["cb_scale"][...] = F.host(sub.cb_scale)
    so["cb_code"][...] = F.host(sub.cb_code)
    del sub
    toks = torch.randint(0, V, (STEPS + 1, B, 1), device="cuda", generator=g, dtype=torch.int32)
    tr = m.set_trace(B * STEPS)
    lg_sel, ng_sel = [], []
    print(f"config[4] {STEPS} decode steps", flush=True)
    for s in range(STEPS):
        lg = m.forward_with_state(toks[s], st)
        ng = m.cb_learn(lg, toks[s + 1, :, 0].contiguous(), st)
        lg_sel.append(F.host(lg)[sel])
        ng_sel.append(F.host(ng)[sel])
    rows = np.concatenate([s * B + np.asarray(sel) for s in range(STEPS)])
    dec_all = F.gpu_decisions(tr, rows)
    m.set_trace(None)
    del tr
    tk = F.host(toks)[:, sel, 0]
    L = cfg["layers"]
    worst = 0.0
    for s in range(STEPS):
        dec = {k: dec_all[k][:, s * len(sel):(s + 1) * len(sel)] for k in ("spikes", "keep", "u", "kth")}
        lo, so, otr = F.forced_oracle(om, tk[s][:, None].astype(np.int32), dec, so)
        no = om.cb_learn(lo, tk[s + 1], so)
        err = float(np.max(np.abs(lg_sel[s] - lo)))
        worst = max(worst, err)
        assert err < 1e-2, (s, err)
        assert F.rel(ng_sel[s], no) < 1e-4, (s, ng_sel[s], no)
        F.check_decisions(cfg, dec, otr, f"config[4] step {s}")
    print(f"config[4]: logits max abs err {worst:.2e} over {STEPS} steps", flush=True)
    sub = st.select(sel)
    F.check_state(so, sub)
    assert F.rel(F.host(sub.cb_tab), so["cb_tab"]) < 1e-4
    assert F.rel(F.host(sub.cb_scale), so["cb_scale"]) < 1e-12
    assert np.max(np.abs(F.host(sub.cb_code) - so["cb_code"])) < 1e-5
    assert L == 8 and st.eng_len == PRE + STEPS
