"""The engram store's cap on the device (ava_engram_evict, evict of gpu/state.rs:518-590) against the
oracle's evict_engram, whose ranking the reference's own cap test pins (tests/test_oracle_engram_count.py):
the same kept slots in store order, moved bit for bit with their counts, for both rules, f32 and fp16
stores, several rounds of the kernel's 256-slot compaction, ties, unseen slots, and the length on the
device; plus the hand-ranked cases of Evict::Oldest and Evict::LeastRead."""
import numpy as np
import pytest
import torch

import oracle.oracle as O
from ava_amd import synth
from ava_amd.model import State

pytestmark = pytest.mark.gpu


def _filled(cfg, B, cap, n, seed, device_len=False):
    st = State(cfg, B, cap, device="cuda", device_len=device_len)
    g = torch.Generator().manual_seed(seed)
    for t in (st.eng_k, st.eng_v):
        t.copy_(torch.randn(t.shape, generator=g, dtype=torch.float64).to(t.dtype))
    st.eng_len, st.seen = n, n
    if device_len:
        st.eng_len_dev.fill_(n)
    return st


def test_evict_keeps_the_last_entries_in_order():
    """Evict::Oldest (state.rs:518-540): the store keeps its last eng_max entries, oldest first."""
    cfg = synth.config("tiny")
    st = _filled(cfg, 2, 20, 13, seed=8)
    k0, v0 = st.eng_k.clone(), st.eng_v.clone()
    st.eng_max = 5
    st.evict()
    torch.cuda.synchronize()
    assert st.eng_len == 5
    assert torch.equal(st.eng_k[:, :5], k0[:, 8:13]) and torch.equal(st.eng_v[:, :5], v0[:, 8:13])
    st.eng_max = 16
    st.evict()  # under the cap: nothing moves
    assert st.eng_len == 5 and torch.equal(st.eng_k[:, :5], k0[:, 8:13])


def test_evict_least_read_ranks_by_reads_per_later_query():
    """Evict::LeastRead (state.rs:540-590): per stream the slots rank by (seen by a later query, reads /
    age, index) and the last eng_max stay, in store order, with their counts; slots no later query
    has seen (age 0) rank last; ties go oldest first."""
    cfg = synth.config("tiny")
    st = _filled(cfg, 2, 20, 10, seed=11)
    k0 = st.eng_k.clone()
    st.eng_rule, st.eng_max = "least-read", 4
    reads = torch.tensor([[5.0, 1.0, 3.0, 0.2, 2.0, 2.0, 9.0, 0.0, 0.0, 0.0],
                          [0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0]], device="cuda")
    age = torch.tensor([[9.0, 8.0, 7.0, 6.0, 4.0, 4.0, 3.0, 2.0, 1.0, 0.0],
                        [9.0, 8.0, 7.0, 6.0, 5.0, 4.0, 3.0, 2.0, 1.0, 0.0]], device="cuda")
    st.eng_reads = torch.zeros((2, 20), device="cuda")
    st.eng_age = torch.zeros((2, 20), device="cuda")
    st.eng_reads[:, :10], st.eng_age[:, :10] = reads, age
    st.evict()
    torch.cuda.synchronize()
    # row 0: reads / age = .556 .125 .429 .033 .5 .5 3 0 0 | unseen slot 9 last; kept: 0, 5 (tie with 4:
    # the older 4 goes first), 6, 9; row 1: all zero reads, so the newest seen slots and the unseen one
    want = [[0, 5, 6, 9], [6, 7, 8, 9]]
    assert st.eng_len == 4
    for r in range(2):
        assert torch.equal(st.eng_k[r, :4], k0[r, want[r]])
        assert torch.equal(st.eng_reads[r, :4], reads[r, want[r]]) and torch.equal(st.eng_age[r, :4], age[r, want[r]])


@pytest.mark.parametrize("rule", ["oldest", "least-read"])
@pytest.mark.parametrize("n,mx,de,half,dlen", [(13, 5, 64, False, False), (300, 200, 64, True, True),
                                               (777, 500, 32, False, True), (1100, 37, 1024, True, False),
                                               (600, 599, 64, False, False)])
def test_evict_matches_the_oracle(rule, n, mx, de, half, dlen):
    """Random stores and counts (a fifth of the slots unseen, a third of the rest sharing one value, so
    the index breaks ties) through the kernel and through the oracle's evict_engram: equal kept keys,
    values and counts, bit for bit; the device length, when kept, becomes eng_max."""
    cfg = dict(synth.config("tiny"), eng_dim=de, eng_half=half)
    B, cap = 3, n + 16
    print(f"evict rule={rule} n={n} max={mx} de={de} half={half} device_len={dlen}", flush=True)
    st = _filled(cfg, B, cap, n, seed=n + mx, device_len=dlen)
    rng = np.random.default_rng(n * 7 + mx)
    age = rng.integers(1, 50, (B, cap)).astype(np.float32)
    age[rng.random((B, cap)) < 0.2] = 0.0
    reads = (rng.random((B, cap)) * age).astype(np.float32)
    tie = rng.random((B, cap)) < 0.33
    reads[tie] = 0.5 * age[tie]
    st.eng_rule, st.eng_max = rule, mx
    st.eng_reads = torch.from_numpy(reads).cuda()
    st.eng_age = torch.from_numpy(age).cuda()
    so = {"eng_k": st.eng_k.cpu().numpy(), "eng_v": st.eng_v.cpu().numpy(), "eng_len": n,
          "eng_reads": reads.copy(), "eng_age": age.copy()}
    O.evict_engram(so, mx, rule)
    st.evict()
    torch.cuda.synchronize()
    assert st.eng_len == so["eng_len"] == mx
    for key in ("eng_k", "eng_v", "eng_reads", "eng_age"):
        assert np.array_equal(getattr(st, key).cpu().numpy()[:, :mx], so[key][:, :mx]), key
    if dlen:
        assert int(st.eng_len_dev.cpu()[0]) == mx
