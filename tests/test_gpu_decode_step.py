"""The overlapped decode step (Model.decode_step, ava_model_decode_step): the previous token's table
step on a second stream while this token's blocks run, against the plain order (cb_learn, then
forward) on a twin state. Everything must be the same bits: the logits of every step, the nats of
every table step, and at the end the table, its scale, the code and the carried state. Then the same
steps as two captured graphs (even and odd steps alternate the logits and next buffers), replayed
with eager work between replays."""
import numpy as np
import pytest
import torch

from ava_amd import synth

pytestmark = pytest.mark.gpu


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


STATE = ("lif_v", "lif_s", "lif_a", "mem_f", "mem_s", "cb_tab", "cb_scale", "cb_code", "eng_k", "eng_v")


def setup(seed, B, prefill, steps, half=True):
    from ava_amd.model import Model
    cfg = synth.config("tiny_cb")
    cfg["eng_half"] = half
    prm = synth.params(cfg, seed=seed)
    V = cfg["vocab"]
    toks = np.random.default_rng(seed + 1).integers(0, V, (B, prefill + steps + 1)).astype(np.int32)
    nexts = toks.copy()
    nexts[1, prefill + 2] = -1  # an ignored next word (outside the vocabulary) for one stream
    m = Model(cfg, prm)
    return cfg, m, toks, nexts


def reference_steps(m, toks, nexts, B, prefill, steps, cap):
    """cb_learn then forward, in order, on one stream."""
    sa = m.state(B, eng_cap=cap, device_len=True)
    pre = torch.from_numpy(np.ascontiguousarray(toks[:, :prefill])).cuda()
    lg = m.forward_with_state(pre, sa)
    last = lg.view(B, prefill, -1)[:, -1]
    logits, nats = [], []
    for t in range(prefill, prefill + steps):
        nxt = torch.from_numpy(np.ascontiguousarray(nexts[:, t])).cuda()
        nats.append(host(m.cb_learn(last, nxt, sa)).copy())
        lg = m.forward_with_state(torch.from_numpy(np.ascontiguousarray(toks[:, t:t + 1])).cuda(), sa)
        logits.append(host(lg).copy())
        last = lg
    nxt = torch.from_numpy(np.ascontiguousarray(nexts[:, prefill + steps])).cuda()
    nats.append(host(m.cb_learn(last, nxt, sa)).copy())
    return sa, logits, nats


def test_decode_step_equals_learn_then_forward():
    B, prefill, steps = 4, 9, 7
    print(f"decode_step B={B} prefill={prefill} steps={steps}", flush=True)
    cfg, m, toks, nexts = setup(21, B, prefill, steps)
    V, cap = cfg["vocab"], prefill + steps
    sa, want_lg, want_nats = reference_steps(m, toks, nexts, B, prefill, steps, cap)

    sb = m.state(B, eng_cap=cap, device_len=True)
    pre = torch.from_numpy(np.ascontiguousarray(toks[:, :prefill])).cuda()
    lg0 = m.forward_with_state(pre, sb)
    prev = lg0.view(B, prefill, V)[:, -1]
    bufs = [torch.empty((B, V), device="cuda") for _ in range(2)]
    nxts = [torch.empty(B, dtype=torch.int32, device="cuda") for _ in range(2)]
    nats = torch.empty(B, dtype=torch.float64, device="cuda")
    for i, t in enumerate(range(prefill, prefill + steps)):
        nxts[i % 2].copy_(torch.from_numpy(np.ascontiguousarray(nexts[:, t])))
        out = bufs[i % 2]
        m.decode_step(torch.from_numpy(np.ascontiguousarray(toks[:, t:t + 1])).cuda(), sb, out, prev, nxts[i % 2], nats)
        assert np.array_equal(host(nats), want_nats[i], equal_nan=True), f"nats, step {i}"
        assert np.array_equal(host(out), want_lg[i]), f"logits, step {i}"
        prev = out
    last = m.cb_learn(prev, torch.from_numpy(np.ascontiguousarray(nexts[:, prefill + steps])).cuda(), sb)
    assert np.array_equal(host(last), want_nats[-1], equal_nan=True)
    assert sb.eng_len == sa.eng_len
    for name in STATE:
        assert np.array_equal(host(getattr(sb, name)), host(getattr(sa, name))), name


def test_decode_step_graphs_equal_learn_then_forward():
    B, prefill, steps = 3, 6, 8
    print(f"decode_step graphs B={B} prefill={prefill} steps={steps}", flush=True)
    cfg, m, toks, nexts = setup(31, B, prefill, steps)
    V, cap = cfg["vocab"], prefill + steps
    sa, want_lg, want_nats = reference_steps(m, toks, nexts, B, prefill, steps, cap)

    sb = m.state(B, eng_cap=cap, device_len=True)
    pre = torch.from_numpy(np.ascontiguousarray(toks[:, :prefill])).cuda()
    lg0 = m.forward_with_state(pre, sb)
    bufs = [torch.empty((B, V), device="cuda") for _ in range(2)]
    nxts = [torch.empty(B, dtype=torch.int32, device="cuda") for _ in range(2)]
    nats = torch.empty(B, dtype=torch.float64, device="cuda")
    ids = torch.empty((B, 1), dtype=torch.int32, device="cuda")
    # step 0 eagerly from the prefill's last rows (allocates what the steps need), into buffer 0
    nxts[0].copy_(torch.from_numpy(np.ascontiguousarray(nexts[:, prefill])))
    ids.copy_(torch.from_numpy(np.ascontiguousarray(toks[:, prefill:prefill + 1])))
    m.decode_step(ids, sb, bufs[0], lg0.view(B, prefill, V)[:, -1], nxts[0], nats)
    assert np.array_equal(host(bufs[0]), want_lg[0])
    # graph p learns from logits buffer p with next buffer p and writes logits buffer 1 - p: step i
    # replays graph (i - 1) % 2
    graphs = [m.capture_decode_step(sb, ids, bufs[1], bufs[0], nxts[0], nats),
              m.capture_decode_step(sb, ids, bufs[0], bufs[1], nxts[1], nats)]
    other = m.state(B, eng_cap=4)
    for i in range(1, steps):
        t = prefill + i
        nxts[(i - 1) % 2].copy_(torch.from_numpy(np.ascontiguousarray(nexts[:, t])))  # the word after t - 1
        ids.copy_(torch.from_numpy(np.ascontiguousarray(toks[:, t:t + 1])))
        graphs[(i - 1) % 2].replay()
        torch.cuda.synchronize()
        assert np.array_equal(host(nats), want_nats[i], equal_nan=True), f"nats, replay {i}"
        assert np.array_equal(host(bufs[i % 2]), want_lg[i]), f"logits, replay {i}"
        m.forward_with_state(ids.clone(), other if i < 4 else m.state(B, eng_cap=4), want_logits=True)
        torch.cuda.synchronize()
    last = m.cb_learn(bufs[(steps - 1) % 2],
                      torch.from_numpy(np.ascontiguousarray(nexts[:, prefill + steps])).cuda(), sb)
    assert np.array_equal(host(last), want_nats[-1], equal_nan=True)
    assert sb.eng_len == sa.eng_len == cap
    for name in STATE:
        assert np.array_equal(host(getattr(sb, name)), host(getattr(sa, name))), name
