"""Calls on different streams of one device use separate scratch memory: the prefill GEMM's
K-piece workspace, the wide GEMV's partial sums and the argmax's per-workgroup bests.
Each check launches the same entry point on two streams back to back, several times,
with different inputs, and compares with one-stream results bit for bit."""
import numpy as np
import pytest
import torch

from kata_amd import ops
from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def _two_streams(dev, fn, args_a, args_b, reps=4):
    s1, s2 = torch.cuda.Stream(dev), torch.cuda.Stream(dev)
    ref_a, ref_b = fn(*args_a), fn(*args_b)           # default stream, one at a time
    torch.cuda.synchronize()
    outs = []
    for _ in range(reps):
        with torch.cuda.stream(s1):
            a = fn(*args_a)
        with torch.cuda.stream(s2):
            b = fn(*args_b)
        outs.append((a, b))
    torch.cuda.synchronize()
    for a, b in outs:
        assert torch.equal(a, ref_a) and torch.equal(b, ref_b)


def test_gemm_pieces_two_streams(dev):
    M, K, N = 512, 1024, 17408                           # 272 tiles: the last 16 split along K
    W = torch.from_numpy(orc.synth_ptq1(N, K, 61)[0]).to(dev)
    A1 = torch.from_numpy(orc.synth_x(M, K, 62)).to(dev)
    A2 = torch.from_numpy(orc.synth_x(M, K, 63)).to(dev)
    _two_streams(dev, lambda A: ops.gemm_ptq1_f16(A, W, K, N), (A1,), (A2,))


def test_wide_two_streams(dev):
    K, N, T = 5120, 17408, 8                            # K split over workgroups
    W = torch.from_numpy(orc.synth_ptq1(N, K, 64)[0]).to(dev)
    x1 = torch.from_numpy(orc.synth_x(T, K, 65)).to(dev)
    x2 = torch.from_numpy(orc.synth_x(T, K, 66)).to(dev)
    _two_streams(dev, lambda x: ops.gemv_ptq1_wide(W, x, K, N), (x1,), (x2,))


def test_argmax_two_streams(dev):
    n = 248320
    rng = np.random.default_rng(67)
    x1 = torch.from_numpy(rng.standard_normal(n).astype(np.float32)).to(dev)
    x2 = torch.from_numpy(rng.standard_normal(n).astype(np.float32)).to(dev)
    _two_streams(dev, lambda x: ops.argmax(x).clone(), (x1,), (x2,))
