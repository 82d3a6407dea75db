"""The non-finite guard (gpu/model/fstep/arch.rs:780-783, 861-864): a stream whose memory inputs hold a
non-finite value is reported by ava_model_nonfinite and its fast weights are left as they were; the
other streams are computed as if it were not there (rows are independent)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.mark.parametrize("T", [1, 5])
def test_nonfinite_memory_input_commits_no_fast_weights(T):
    from ava_amd import synth
    from ava_amd.model import Model
    cfg = synth.config("tiny")
    prm = synth.params(cfg, seed=21)
    bad_id = cfg["vocab"] - 1
    prm["tok_emb"] = np.array(prm["tok_emb"], np.float32, copy=True)
    prm["tok_emb"][bad_id] = np.nan  # this token's embedding poisons every block of its stream
    print(f"guard T={T}", flush=True)
    m = Model(cfg, prm)
    rng = np.random.default_rng(3)
    B = 3
    st = m.state(B, eng_cap=64)
    warm = torch.from_numpy(rng.integers(0, bad_id, (B, 8)).astype(np.int32)).cuda()
    m.forward_with_state(warm, st)
    assert m.nonfinite() == []
    F0, S0 = host(st.mem_f).copy(), host(st.mem_s).copy()
    assert np.all(np.isfinite(F0))

    ids = rng.integers(0, bad_id, (B, T)).astype(np.int32)
    clean = ids.copy()
    ids[1, T // 2] = bad_id
    # the same call on a copy of the state with stream 1's clean ids: streams 0 and 2 must agree
    st2 = st.select([0, 1, 2])
    lg = host(m.forward_with_state(torch.from_numpy(ids).cuda(), st)).reshape(B, T, -1)
    assert m.nonfinite() == [1]
    lg2 = host(m.forward_with_state(torch.from_numpy(clean).cuda(), st2)).reshape(B, T, -1)
    assert m.nonfinite() == []
    F, S = host(st.mem_f), host(st.mem_s)
    # stream 1: every block's fast weights as before the call
    assert np.array_equal(F[:, 1], F0[:, 1]) and np.array_equal(S[:, 1], S0[:, 1])
    # streams 0 and 2: the same as without the poisoned token
    for b in (0, 2):
        assert np.array_equal(lg[b], lg2[b])
        assert np.array_equal(F[:, b], host(st2.mem_f)[:, b])
    # and their fast weights moved
    assert not np.array_equal(F[:, 0], F0[:, 0])


def test_refused_forward_reports_no_rows_of_an_earlier_one():
    """A forward refused by its checks (here: the engram store is full) after one that marked a stream
    reports no streams, and a rows buffer smaller than the last forward's streams is refused."""
    import ctypes as C
    from ava_amd import synth
    from ava_amd._lib import lib
    from ava_amd.model import Model
    cfg = synth.config("tiny")
    prm = synth.params(cfg, seed=22)
    bad_id = cfg["vocab"] - 1
    prm["tok_emb"] = np.array(prm["tok_emb"], np.float32, copy=True)
    prm["tok_emb"][bad_id] = np.nan
    print("guard refused forward", flush=True)
    m = Model(cfg, prm)
    st = m.state(4, eng_cap=8)
    ids = np.zeros((4, 4), np.int32)
    ids[3, 1] = bad_id
    m.forward_with_state(torch.from_numpy(ids).cuda(), st)
    assert m.nonfinite() == [3]
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    rows, n = (C.c_int32 * 2)(), C.c_int(0)
    assert lib().ava_model_nonfinite(m.h, rows, 2, C.byref(n), stream) != 0  # 2 < the 4 streams
    small = m.state(2, eng_cap=4)
    with pytest.raises(RuntimeError):  # 8 > the 4 entries the store holds: refused before it runs
        m.forward_with_state(torch.zeros((2, 8), dtype=torch.int32, device="cuda"), small)
    assert m.nonfinite() == []
    assert lib().ava_model_nonfinite(m.h, rows, 2, C.byref(n), stream) == 0 and n.value == 0
