"""fgs_inclusive_scan_u32_noalloc: the allocation-free variant of
fgs_inclusive_scan_u32, whose state lives in the library's static device
array.  Through the C ABI it must give the workspace entry point's results bit
for bit, on two calls in a row (the second smaller, so the first call's
published chunk states are still in the array), and reject sizes above its
maximum with a clear error."""
import ctypes

import numpy as np
import pytest

from fastgs_core_amd import _lib

pytestmark = pytest.mark.gpu


def _say(*a):
    print("[gpu-test] no-alloc scan", *a, flush=True)


def test_noalloc_scan_matches_workspace_scan_twice():
    import torch

    lib = _lib.load()
    dev = torch.device("cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    rng = np.random.default_rng(0)
    for n in (3_000_001, 70_001):
        _say("n =", n)
        x = rng.integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32)
        xin = torch.from_numpy(x.view(np.int32)).to(dev)
        ref = torch.empty(n, dtype=torch.int32, device=dev)
        got = torch.full((n,), -1, dtype=torch.int32, device=dev)
        ws = torch.empty(int(lib.fgs_scan_workspace_bytes(n)), dtype=torch.uint8, device=dev)
        status = torch.full((2,), -1, dtype=torch.int32, device=dev)
        _lib.check(lib.fgs_inclusive_scan_u32(xin.data_ptr(), ref.data_ptr(), n, ws.data_ptr(),
                                              status.data_ptr(), stream))
        _lib.check(lib.fgs_inclusive_scan_u32_noalloc(xin.data_ptr(), got.data_ptr(), n,
                                                      status[1:].data_ptr(), stream))
        torch.cuda.synchronize()
        g = got.cpu().numpy().view(np.uint32)
        np.testing.assert_array_equal(g, ref.cpu().numpy().view(np.uint32))
        np.testing.assert_array_equal(g, np.cumsum(x, dtype=np.uint64).astype(np.uint32))
        assert status.cpu().tolist() == [0, 0]  # every wait completed


def test_noalloc_scan_rejects_sizes_above_its_maximum():
    lib = _lib.load()
    rc = lib.fgs_inclusive_scan_u32_noalloc(None, None, (1 << 28) + 1, None, None)
    assert rc == -1
    assert b"exceeds the maximum" in lib.fgs_last_error()
    assert lib.fgs_inclusive_scan_u32_noalloc(None, None, 0, None, None) == 0
