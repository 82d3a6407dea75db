"""A decode step captured as a HIP graph (Model.capture_decode) against the same steps run eagerly.

The captured forward reads the engram store's length from the device and advances it there, so
every replay is a new token. Replays are checked one by one against the eager steps (the same
kernels and launch shapes: the same bits), with eager work and synchronizations between replays, as
graph replays that go wrong tend to do so after the first one. While the graph lives the model's
scratch is frozen: a forward that would need more is refused on the host (nothing is freed under
the graph)."""
import numpy as np
import pytest
import torch

from ava_amd import synth
from ava_amd._lib import AvaError

pytestmark = pytest.mark.gpu


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def test_decode_graph_replays_equal_eager_steps():
    from ava_amd.model import Model
    cfg = synth.config("tiny_cb")
    cfg["eng_half"] = True
    prm = synth.params(cfg, seed=11)
    B, prefill, steps = 3, 20, 6
    V = cfg["vocab"]
    toks = np.random.default_rng(12).integers(0, V, (B, prefill + steps + 1)).astype(np.int32)
    cap = prefill + steps
    print(f"decode graph B={B} prefill={prefill} steps={steps}", flush=True)
    m = Model(cfg, prm)
    sa = m.state(B, eng_cap=cap, device_len=True)
    sb = m.state(B, eng_cap=cap, device_len=True)
    pre = torch.from_numpy(np.ascontiguousarray(toks[:, :prefill])).cuda()
    m.forward_with_state(pre, sa, want_logits=False)
    m.forward_with_state(pre, sb, want_logits=False)
    col = lambda t: torch.from_numpy(np.ascontiguousarray(toks[:, t:t + 1])).cuda()
    nxt = lambda t: torch.from_numpy(np.ascontiguousarray(toks[:, t + 1])).cuda()

    # eager reference steps on state a
    want = []
    for t in range(prefill, prefill + steps):
        lg = m.forward_with_state(col(t), sa)
        nats = m.cb_learn(lg, nxt(t), sa)
        want.append((host(lg).copy(), host(nats).copy()))

    # state b: the first step eagerly (allocates), then capture over fixed buffers and replay
    ids_buf = col(prefill).clone()
    nxt_buf = nxt(prefill).clone()
    lg_buf = torch.empty((B, V), device="cuda")
    nats_buf = torch.empty(B, dtype=torch.float64, device="cuda")
    m.forward_with_state(ids_buf, sb, lg_buf)
    m.cb_learn(lg_buf, nxt_buf, sb, nats=nats_buf)
    assert np.array_equal(host(lg_buf), want[0][0])
    g = m.capture_decode(sb, ids_buf, lg_buf, nxt_buf, nats_buf)
    other = m.state(B, eng_cap=4)
    for i, t in enumerate(range(prefill + 1, prefill + steps)):
        ids_buf.copy_(col(t))
        nxt_buf.copy_(nxt(t))
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(host(lg_buf), want[i + 1][0]), f"replay {i}"
        assert np.array_equal(host(nats_buf), want[i + 1][1]), f"replay {i}"
        # eager work between replays: a forward of the same size on another state
        m.forward_with_state(col(t).clone(), other if i < 3 else m.state(B, eng_cap=4), want_logits=True)
        torch.cuda.synchronize()
    assert sb.eng_len == sa.eng_len == cap
    assert int(host(sb.eng_len_dev)[0]) == cap
    for name in ("lif_v", "lif_s", "mem_f", "mem_s", "cb_tab", "cb_scale", "eng_k", "eng_v"):
        assert np.array_equal(host(getattr(sb, name)), host(getattr(sa, name))), name
    # the store is full: a further replay is refused on the host
    with pytest.raises(ValueError):
        g.replay()
    # frozen scratch: a larger batch is refused before anything is launched
    big = m.state(2 * B, eng_cap=4)
    with pytest.raises(AvaError):
        m.forward_with_state(torch.zeros((2 * B, 4), dtype=torch.int32, device="cuda"), big)


def test_capped_decode_graph_evicts_on_replay():
    """A capped store (eng_max, oldest first) under a captured decode step: the eviction runs inside the
    graph on the device length, so replays past the cap keep going, and every replay equals the eager
    step (the same kernels: the same bits); the stores and device lengths agree at the end."""
    from ava_amd.model import Model
    cfg = synth.config("tiny")
    prm = synth.params(cfg, seed=21)
    B, prefill, steps, mx = 2, 12, 8, 14
    V = cfg["vocab"]
    toks = np.random.default_rng(22).integers(0, V, (B, prefill + steps + 1)).astype(np.int32)
    print(f"capped decode graph B={B} prefill={prefill} steps={steps} max={mx}", flush=True)
    m = Model(cfg, prm)
    sa = m.state(B, eng_cap=mx + prefill, eng_max=mx, device_len=True)
    sb = m.state(B, eng_cap=mx + prefill, eng_max=mx, device_len=True)
    pre = torch.from_numpy(np.ascontiguousarray(toks[:, :prefill])).cuda()
    m.forward_with_state(pre, sa, want_logits=False)
    m.forward_with_state(pre, sb, want_logits=False)
    col = lambda t: torch.from_numpy(np.ascontiguousarray(toks[:, t:t + 1])).cuda()
    want = [host(m.forward_with_state(col(t), sa)).copy() for t in range(prefill, prefill + steps)]
    assert sa.eng_len == mx and int(host(sa.eng_len_dev)[0]) == mx

    ids_buf = col(prefill).clone()
    lg_buf = torch.empty((B, V), device="cuda")
    m.forward_with_state(ids_buf, sb, lg_buf)
    assert np.array_equal(host(lg_buf), want[0])
    g = m.capture_decode(sb, ids_buf, lg_buf)
    for i, t in enumerate(range(prefill + 1, prefill + steps)):
        ids_buf.copy_(col(t))
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(host(lg_buf), want[i + 1]), f"replay {i}"
        m.forward_with_state(col(t).clone(), m.state(B, eng_cap=4), want_logits=True)
        torch.cuda.synchronize()
    assert sb.eng_len == sa.eng_len == mx
    assert int(host(sb.eng_len_dev)[0]) == mx
    for name in ("eng_k", "eng_v", "mem_f", "lif_v"):
        assert np.array_equal(host(getattr(sb, name))[:, :mx] if name.startswith("eng") else host(getattr(sb, name)),
                              host(getattr(sa, name))[:, :mx] if name.startswith("eng") else host(getattr(sa, name))), name
    # the least-read rule's counts take the length from the host: its capture is refused
    sc = m.state(B, eng_cap=mx + prefill, eng_max=mx, eng_rule="least-read", device_len=True)
    with pytest.raises(ValueError):
        m.capture_decode(sc, ids_buf, lg_buf)
