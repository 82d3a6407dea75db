"""ava_q8_matmul_noalloc (no reference counterpart: the product for callers that cannot allocate)
against ava_q8_matmul with a caller workspace, through the C ABI: the same bits on two calls in a
row, the second with fewer rows (the shared scratch keeps the first call's contents), and a size
beyond the library's scratch refused with a status before anything runs on the GPU."""
import ctypes as C

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _stream():
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def test_noalloc_product_equals_workspace_product():
    from ava_amd import ops
    from ava_amd._lib import lib
    L = lib()
    rng = np.random.default_rng(31)
    din, dout = 1024, 1536
    w = ops.QW.from_tensor(torch.from_numpy((rng.standard_normal((din, dout)) * 0.02).astype(np.float32)).cuda())
    for m, planes in ((2048, 3), (300, 3), (77, 1)):
        print(f"noalloc m={m} din={din} dout={dout} planes={planes}", flush=True)
        x = torch.from_numpy(rng.standard_normal((m, din)).astype(np.float32)).cuda()
        want = ops.mm(x, w, planes=planes)
        got = torch.full((m, dout), float("nan"), device="cuda")
        rc = L.ava_q8_matmul_noalloc(C.c_void_p(x.data_ptr()), m, C.byref(w.c), planes, C.c_void_p(got.data_ptr()),
                                     _stream())
        assert rc == 0, L.ava_last_error()
        torch.cuda.synchronize()
        assert np.array_equal(got.cpu().numpy().view(np.uint32), want.cpu().numpy().view(np.uint32))


def test_noalloc_refuses_sizes_beyond_its_scratch():
    from ava_amd import ops
    from ava_amd._lib import lib
    L = lib()
    w = ops.QW.from_tensor(torch.zeros((4096, 64), device="cuda"))
    m = 4096  # 3 planes x 4096 rows x 4096 inputs = 48 MiB > 32 MiB
    assert L.ava_q8_workspace(m, 4096, 3) > 32 << 20
    y = torch.empty((m, 64), device="cuda")
    rc = L.ava_q8_matmul_noalloc(C.c_void_p(y.data_ptr()), m, C.byref(w.c), 3, C.c_void_p(y.data_ptr()), _stream())
    assert rc == 2 and b"scratch" in L.ava_last_error()
