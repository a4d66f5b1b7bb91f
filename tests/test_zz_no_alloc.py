"""The no-allocation wide verification GEMV (kata_gemv_ptq1_wide_noalloc) through the C ABI:
the same results as kata_gemv_ptq1_wide bit for bit, and the oracle's within the GEMV bar,
on two calls in a row, the second with a smaller input (the shared scratch keeps the first
call's contents); rejected sizes fail cleanly."""
import ctypes

import numpy as np
import pytest
import torch

from kata_amd.capi import lib
from oracle import oracle as orc
from tests.conftest import rel_l2

pytestmark = pytest.mark.gpu


def _call(fn, W, x, y, K, N, T):
    rc = fn(ctypes.c_void_p(W.data_ptr()), ctypes.c_void_p(x.data_ptr()), 1 if x.dtype == torch.float16 else 0,
            ctypes.c_void_p(y.data_ptr()), K, N, T, None)
    assert rc == 0, lib().kata_last_error().decode()


@pytest.mark.parametrize("dt", [torch.float16, torch.float32])
def test_noalloc_matches_wide(dev, dt):
    L = lib()
    assert L.kata_gemv_ptq1_wide_noalloc_scratch_bytes() == 4 << 20
    # first call large (several K chunks, rows over several launches of the 4 MiB scratch),
    # second smaller (fewer rows, other K, other T)
    for K, N, T in ((5120, 248320, 8), (17408, 5120, 5), (1024, 700, 3)):
        W_np, _, _ = orc.synth_ptq1(N, K, K + N + T)
        x_np = orc.synth_x(T, K, K + T)
        W = torch.from_numpy(W_np).to(dev)
        x = torch.from_numpy(x_np).to(dev).to(dt)
        y0 = torch.full((T, N), float("nan"), device=dev)
        y1 = torch.full((T, N), float("nan"), device=dev)
        _call(L.kata_gemv_ptq1_wide, W, x, y0, K, N, T)
        _call(L.kata_gemv_ptq1_wide_noalloc, W, x, y1, K, N, T)
        torch.cuda.synchronize()
        assert torch.equal(y0, y1), (K, N, T)
        rows = np.arange(0, N, max(1, N // 97))
        ref = orc.gemv_ptq1(np.ascontiguousarray(W_np[rows]), x.float().cpu().numpy(), K, len(rows), T)
        assert rel_l2(y1.cpu().numpy()[:, rows], ref).max() < 2e-4


def test_noalloc_rejects(dev):
    L = lib()
    W = torch.zeros(28, dtype=torch.uint8, device=dev)
    x = torch.zeros((8, 128), dtype=torch.float16, device=dev)
    y = torch.zeros((8, 1), device=dev)
    rc = L.kata_gemv_ptq1_wide_noalloc(ctypes.c_void_p(W.data_ptr()), ctypes.c_void_p(x.data_ptr()), 1,
                                       ctypes.c_void_p(y.data_ptr()), 100, 1, 8, None)
    assert rc == -1 and b"multiple of 128" in L.kata_last_error()
    rc = L.kata_gemv_ptq1_wide_noalloc(ctypes.c_void_p(W.data_ptr()), ctypes.c_void_p(x.data_ptr()), 1,
                                       ctypes.c_void_p(y.data_ptr()), 128, 1, 9, None)
    assert rc == -1
