"""GPU parity of the PTQ1_0 decode GEMV (T=1, T=2) against the CPU oracle.

Contract: relative L2 error <= 1e-3 per output vector (fp32-accumulated outputs).
The kernel's only approximation is the 16-bit block-fixed-point activation, so the
observed error is ~1e-5; the tests also bound it tighter (2e-4) to catch a regression
that would still pass the contract by luck.
"""
import numpy as np
import pytest
import torch

from kata_amd import ops
from oracle import oracle as orc
from tests.conftest import rel_l2

pytestmark = pytest.mark.gpu
TOL = 1e-3
TIGHT = 2e-4


def _run(dev, W_np, x_np, K, N, T, half2=False):
    W = torch.from_numpy(W_np).to(dev)
    if half2:
        x = torch.from_numpy(np.ascontiguousarray(x_np.T)).to(dev)        # [K][2]
    else:
        x = torch.from_numpy(x_np).to(dev)
    y = ops.gemv_ptq1(W, x, K, N, T, half2=half2)
    torch.cuda.synchronize()
    return y.cpu().numpy()


def test_golden_t1_t2(dev, golden):
    K, N = int(golden["ptq1_K"]), int(golden["ptq1_N"])
    x = golden["gemv_x"]
    for T in (1, 2):
        y = _run(dev, golden["ptq1_W"], np.ascontiguousarray(x[:T]), K, N, T)
        assert rel_l2(y, golden["gemv_y"][:T]).max() < TIGHT
        assert y[0, 5] == 0.0                          # all-zero trit row is exactly zero


@pytest.mark.parametrize("K,N,T,dtype", [
    (128, 16, 1, np.float16), (128, 1, 1, np.float32), (256, 17, 2, np.float16),
    (640, 33, 1, np.float32), (1024, 64, 2, np.float32), (5120, 80, 1, np.float16),
    (6144, 48, 2, np.float16), (17408, 32, 1, np.float16), (17408, 20, 2, np.float32),
    (-2, 16, 2, np.float16), (-1, 16, 1, np.float32),      # largest K per T (LDS bound)
])
def test_random_vs_oracle(dev, K, N, T, dtype):
    if K < 0:
        from kata_amd.capi import lib
        K = lib().kata_gemv_ptq1_max_k(-K)
    seed = K * 131 + N * 7 + T
    W, _, _ = orc.synth_ptq1(N, K, seed)
    x = orc.synth_x(T, K, seed + 1, dtype)
    y = _run(dev, W, x, K, N, T)
    ref = orc.gemv_ptq1(W, x.astype(np.float32), K, N, T)
    err = rel_l2(y, ref)
    print(f"K={K} N={N} T={T} {np.dtype(dtype).name}: max rel L2 {err.max():.2e}")
    assert err.max() < TIGHT


def test_half2_layout_matches_rows(dev):
    K, N = 5120, 96
    W, _, _ = orc.synth_ptq1(N, K, 3)
    x = orc.synth_x(2, K, 4)
    y_rows = _run(dev, W, x, K, N, 2)
    y_ilv = _run(dev, W, x, K, N, 2, half2=True)
    assert np.array_equal(y_rows, y_ilv)


def test_t2_rows_equal_t1(dev):
    """Each token of a T=2 call is quantised and reduced exactly as a T=1 call on it."""
    K, N = 5120, 256
    W_np, _, _ = orc.synth_ptq1(N, K, 5)
    x = torch.from_numpy(orc.synth_x(2, K, 6)).to(dev)
    W = torch.from_numpy(W_np).to(dev)
    y2 = ops.gemv_ptq1(W, x, K, N, 2)
    for t in range(2):
        y1 = ops.gemv_ptq1(W, x[t:t + 1].contiguous(), K, N, 1)
        torch.cuda.synchronize()
        assert torch.equal(y1[0], y2[t])


def test_special_inputs(dev):
    K, N = 1024, 48
    W_np, t, s = orc.synth_ptq1(N, K, 7)
    W = torch.from_numpy(W_np).to(dev)
    # zero activation -> exactly zero
    y = ops.gemv_ptq1(W, torch.zeros((1, K), dtype=torch.float16, device=dev), K, N, 1)
    assert torch.count_nonzero(y).item() == 0
    # x = 1 -> d * sum(t) per block
    y = ops.gemv_ptq1(W, torch.ones((1, K), dtype=torch.float32, device=dev), K, N, 1).cpu().numpy()
    want = (t.reshape(N, K // 128, 128).sum(-1) * s.astype(np.float64)).sum(-1)
    assert rel_l2(y, want[None]).max() < TIGHT
    # wide dynamic range inside blocks (one large element per block)
    x = orc.synth_x(1, K, 8, np.float32)
    x[0, ::128] *= 1000.0
    y = _run(dev, W_np, x, K, N, 1)
    assert rel_l2(y, orc.gemv_ptq1(W_np, x, K, N, 1)).max() < TOL


def test_full_shape_17408x5120(dev):
    """BASELINE config 1 shape: parity on sampled rows vs the oracle, and every row vs a
    torch fp32 product of the GPU-expanded (bit-exact) weights."""
    K, N = 5120, 17408
    W_np, _, _ = orc.synth_ptq1(N, K, 2026)
    x_np = orc.synth_x(2, K, 2027)
    W = torch.from_numpy(W_np).to(dev)
    x = torch.from_numpy(x_np).to(dev)
    for T in (1, 2):
        y = ops.gemv_ptq1(W, x[:T].contiguous(), K, N, T)
        Wexp = ops.expand_f16(W, K, N)
        ref = (x[:T].float() @ Wexp.float().T)
        torch.cuda.synchronize()
        err = rel_l2(y.cpu().numpy(), ref.cpu().numpy())
        assert err.max() < TIGHT, err.max()
        rows = np.arange(0, N, 97)
        sub = np.ascontiguousarray(W_np[rows])
        ref_o = orc.gemv_ptq1(sub, x_np[:T].astype(np.float32), K, len(rows), T)
        assert rel_l2(y.cpu().numpy()[:, rows], ref_o).max() < TIGHT


@pytest.mark.parametrize("K,T", [(1024, 1), (2048, 1), (2048, 2), (3072, 1), (3072, 2), (4096, 1), (4096, 2),
                                 (5120, 1), (5120, 2)])
def test_long_single_matrix_orders(dev, K, T):
    """One matrix of >= 64 tiles per workgroup (66000 rows): the launch picks the tile-strided
    order where its scratch stores fit (K = 3072..5120, and 2048 at T = 1) and the run order
    elsewhere (K = 1024, and 2048 at T = 2, whose strided pair slots would reach past the
    scratch area into the item sums).  Every row against a torch fp32 product of the GPU-expanded weights, sampled
    rows against the oracle."""
    N = 66000
    W_np, _, _ = orc.synth_ptq1(N, K, K + T)
    x_np = orc.synth_x(T, K, K + T + 1)
    W = torch.from_numpy(W_np).to(dev)
    x = torch.from_numpy(x_np).to(dev)
    y = ops.gemv_ptq1(W, x, K, N, T)
    ref = x.float() @ ops.expand_f16(W, K, N).float().T
    torch.cuda.synchronize()
    assert rel_l2(y.cpu().numpy(), ref.cpu().numpy()).max() < TIGHT
    rows = np.arange(0, N, 331)
    ref_o = orc.gemv_ptq1(np.ascontiguousarray(W_np[rows]), x_np.astype(np.float32), K, len(rows), T)
    assert rel_l2(y.cpu().numpy()[:, rows], ref_o).max() < TIGHT


@pytest.mark.parametrize("K,Ns,T,half2", [
    (5120, (96, 8, 8), 1, False), (6144, (40, 13), 2, True), (1024, (5, 64, 3, 17), 2, False),
    (17408, (20,), 1, False),
])
def test_batch_equals_single_calls(dev, K, Ns, T, half2):
    """One launch over several matrices sharing x gives exactly the per-matrix results."""
    Ws_np = [orc.synth_ptq1(N, K, 100 + i)[0] for i, N in enumerate(Ns)]
    x_np = orc.synth_x(T, K, 99)
    x = torch.from_numpy(np.ascontiguousarray(x_np.T) if half2 else x_np).to(dev)
    Ws = [torch.from_numpy(w).to(dev) for w in Ws_np]
    ys = ops.gemv_ptq1_batch(Ws, x, K, list(Ns), T, half2=half2)
    for W, W_np, N, yb in zip(Ws, Ws_np, Ns, ys):
        y1 = ops.gemv_ptq1(W, x, K, N, T, half2=half2)
        torch.cuda.synchronize()
        assert torch.equal(yb, y1)
        ref = orc.gemv_ptq1(W_np, x_np.astype(np.float32), K, N, T)
        assert rel_l2(yb.cpu().numpy(), ref).max() < TIGHT


@pytest.mark.parametrize("K", [3072, 4096, 5120])
def test_strided_short_last_range(dev, K):
    """Tile-strided launch whose last workgroup gets a single, ragged tile: 65283 rows are
    16321 tiles, 64 per workgroup on 256 CUs, so workgroup 255 holds one 3-row tile (fewer
    tiles than the order's phases: most of its waves get no items).  Every row against a
    torch fp32 product of the GPU-expanded weights, sampled rows and the last rows against
    the oracle."""
    N, T = 65283, 1
    W_np, _, _ = orc.synth_ptq1(N, K, K + 7)
    x_np = orc.synth_x(T, K, K + 8)
    W = torch.from_numpy(W_np).to(dev)
    x = torch.from_numpy(x_np).to(dev)
    y = ops.gemv_ptq1(W, x, K, N, T)
    ref = x.float() @ ops.expand_f16(W, K, N).float().T
    torch.cuda.synchronize()
    assert rel_l2(y.cpu().numpy(), ref.cpu().numpy()).max() < TIGHT
    rows = np.concatenate([np.arange(0, N, 509), np.arange(N - 9, N)])
    ref_o = orc.gemv_ptq1(np.ascontiguousarray(W_np[rows]), x_np.astype(np.float32), K, len(rows), T)
    got = y.cpu().numpy()[:, rows]
    assert rel_l2(got, ref_o).max() < TIGHT
    assert np.abs(got[:, -9:] - ref_o[:, -9:]).max() <= 2e-4 * np.abs(ref_o[:, -9:]).max()
