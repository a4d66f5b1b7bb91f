"""lm_head step (src/engine.cpp:191-192): the 248320 x 5120 PTQ1_0 GEMV and the greedy argmax
of its logits (k_argmax, shaders/ops.metal:66-78)."""
import numpy as np
import pytest
import torch

from kata_amd import ops
from oracle import oracle as orc

from conftest import rel_l2

pytestmark = pytest.mark.gpu
INT_MAX = 0x7fffffff


@pytest.fixture(scope="module")
def dev():
    return torch.device("cuda:0")


def ref_argmax(x):
    """The reference loop: an element counts only if strictly greater than the best so far
    (NaN and -inf never do), lowest index on ties, INT_MAX if none counts."""
    v = np.where(np.isnan(x), -np.inf, x)
    m = v.max()
    return INT_MAX if m == -np.inf else int(np.flatnonzero(v == m)[0])


@pytest.mark.parametrize("n", [1, 5, 1023, 4099, 248320])
def test_argmax_random_and_repeated(dev, n):
    rng = np.random.default_rng(n)
    for rep in range(3):                          # the completion counter resets between calls
        x = rng.standard_normal(n).astype(np.float32)
        assert ops.argmax(torch.from_numpy(x).to(dev)).item() == ref_argmax(x)


def test_argmax_ties_nan_inf(dev):
    n = 100003
    x = np.full(n, -1.0, np.float32)
    x[[777, 5000, 99999]] = 3.0                   # tie: lowest index
    x[[10, 20000]] = np.nan                       # NaN never counts
    assert ops.argmax(torch.from_numpy(x).to(dev)).item() == 777
    x[4242] = np.inf
    assert ops.argmax(torch.from_numpy(x).to(dev)).item() == 4242
    y = np.full(n, -np.inf, np.float32)
    y[5] = np.nan
    assert ops.argmax(torch.from_numpy(y).to(dev)).item() == INT_MAX


def test_lm_head_gemv_then_argmax(dev):
    K, N = 5120, 248320
    W_np, _, _ = orc.synth_ptq1(N, K, 4040)
    W = torch.from_numpy(W_np).to(dev)
    x = torch.from_numpy(orc.synth_x(1, K, 4041, np.float32)).to(dev)
    y = ops.gemv_ptq1(W, x, K, N, 1)
    rows = np.r_[0:256, N - 256:N]
    ref = orc.gemv_ptq1(np.ascontiguousarray(W_np[rows]), x.cpu().numpy(), K, len(rows), 1)
    assert rel_l2(y.cpu().numpy()[:, rows], ref).max() < 2e-4
    assert ops.argmax(y).item() == ref_argmax(y.cpu().numpy()[0])


def test_lm_head_strided_order_equals_run_order(dev):
    """The 248320-row lm_head alone runs the tile-strided work order; inside a two-matrix
    batch it runs the contiguous one: the same items and slots, so the same result bit for bit."""
    K, N = 5120, 248320
    gen = torch.Generator(device=dev)
    gen.manual_seed(11)
    nb = K // 128
    blk = torch.empty((N, nb, 28), dtype=torch.uint8, device=dev)
    blk[:, :, :24] = torch.randint(0, 243, (N, nb, 24), generator=gen, device=dev, dtype=torch.uint8)
    blk[:, :, 24:26] = torch.randint(0, 81, (N, nb, 2), generator=gen, device=dev, dtype=torch.uint8)
    blk[:, :, 26:28] = (torch.randn((N, nb), generator=gen, device=dev) * 0.02).abs().half() \
        .view(torch.uint8).view(N, nb, 2)
    W = blk.view(N, nb * 28)
    W2 = W[:64].clone()
    x = torch.randn((1, K), generator=gen, device=dev).half()
    y = ops.gemv_ptq1(W, x, K, N, 1)
    yb, _ = ops.gemv_ptq1_batch([W, W2], x, K, [N, 64], 1)
    assert torch.equal(y, yb)
