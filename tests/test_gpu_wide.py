"""GPU parity of the wide verification GEMV (T = 1..8 token rows, Engine::dWide,
src/engine.cpp:542-556; shaders/wide.metal:41-99) against the CPU oracle.

Contract: relative L2 error <= 1e-3 per output vector; the kernel's only approximation is
the 16-bit block-fixed-point activation, so the tests hold it to 2e-4.  Token rows are
independent: row t of a T-row call (T >= 3) equals the same token in any other such call
bit for bit (the per-(block, token) quantisation and the summation order do not depend on
T); T = 1, 2 run the decode GEMV.  The batch form (1..4 matrices sharing the rows, one
launch) equals single calls bit for bit."""
import numpy as np
import pytest
import torch

from kata_amd import ops
from oracle import oracle as orc
from tests.conftest import rel_l2

pytestmark = pytest.mark.gpu
TIGHT = 2e-4


def test_wide_golden(dev, golden):
    K, N = int(golden["ptq1_K"]), int(golden["ptq1_N"])
    W = torch.from_numpy(golden["ptq1_W"]).to(dev)
    x = torch.from_numpy(np.ascontiguousarray(golden["gemv_x"])).to(dev)
    y = ops.gemv_ptq1_wide(W, x, K, N).cpu().numpy()
    assert rel_l2(y, golden["gemv_y"][: x.shape[0]]).max() < TIGHT
    assert (y[:, 5] == 0.0).all()                      # all-zero trit row is exactly zero


@pytest.mark.parametrize("K,N,T,dtype", [
    (128, 1, 1, np.float16), (256, 17, 3, np.float32), (1024, 130, 8, np.float16),
    (1536, 129, 5, np.float16),            # 12 blocks: one chunk
    (1664, 200, 8, np.float32),            # 13 blocks: two chunks, ragged last chunk
    (5120, 1000, 8, np.float16), (6144, 300, 7, np.float16),
    (17408, 160, 8, np.float16),           # 136 blocks over many chunks
])
def test_wide_vs_oracle(dev, K, N, T, dtype):
    seed = K * 17 + N * 3 + T
    W_np, _, _ = orc.synth_ptq1(N, K, seed)
    x_np = orc.synth_x(T, K, seed + 1, dtype)
    y = ops.gemv_ptq1_wide(torch.from_numpy(W_np).to(dev), torch.from_numpy(x_np).to(dev), K, N).cpu().numpy()
    ref = orc.gemv_ptq1(W_np, x_np.astype(np.float32), K, N, T)
    err = rel_l2(y, ref)
    print(f"K={K} N={N} T={T} {np.dtype(dtype).name}: max rel L2 {err.max():.2e}")
    assert err.max() < TIGHT


def test_wide_rows_independent_and_deterministic(dev):
    """Row t of an 8-row call equals, bit for bit, the same token in a 3-row call at another
    position (the K split, the per-(block, token) quantisation and the summation order do
    not depend on T or the row); T = 1, 2 run the decode GEMV and equal it bit for bit."""
    K, N, T = 5120, 3000, 8
    W_np, _, _ = orc.synth_ptq1(N, K, 5)
    x_np = orc.synth_x(T, K, 6)
    x_np[3] *= 1e3                                     # scales differ per token
    x_np[6, :128] = 0.0                                # an all-zero block of one token
    W = torch.from_numpy(W_np).to(dev)
    x = torch.from_numpy(x_np).to(dev)
    y = ops.gemv_ptq1_wide(W, x, K, N)
    y2 = ops.gemv_ptq1_wide(W, x, K, N)
    assert torch.equal(y, y2)
    for t in range(T):
        x3 = torch.stack([x[(t + 1) % T], x[(t + 2) % T], x[t]]).contiguous()
        y3 = ops.gemv_ptq1_wide(W, x3, K, N)
        assert torch.equal(y[t], y3[2]), t
    for T2 in (1, 2):
        yw = ops.gemv_ptq1_wide(W, x[:T2].contiguous(), K, N)
        yd = ops.gemv_ptq1(W, x[:T2].contiguous(), K, N, T2)
        assert torch.equal(yw, yd)
        assert rel_l2(y[:T2].cpu().numpy(), yd.cpu().numpy()).max() < 1e-6


@pytest.mark.parametrize("K,N", [(5120, 17408), (17408, 5120)])
def test_wide_full_shapes_t8(dev, K, N):
    """The FFN shapes at T = 8 (the reference's kMaxVerify) vs the oracle on sampled rows
    and every row vs a torch fp32 product of the GPU-expanded (bit-exact) weights."""
    W_np, _, _ = orc.synth_ptq1(N, K, K + N)
    x_np = orc.synth_x(8, K, 99)
    W = torch.from_numpy(W_np).to(dev)
    x = torch.from_numpy(x_np).to(dev)
    y = ops.gemv_ptq1_wide(W, x, K, N)
    ref = (x.float() @ ops.expand_f16(W, K, N).float().T)
    err = rel_l2(y.cpu().numpy(), ref.cpu().numpy())
    assert err.max() < TIGHT, err.max()
    rows = np.arange(0, N, 61)
    ref_o = orc.gemv_ptq1(np.ascontiguousarray(W_np[rows]), x_np.astype(np.float32), K, len(rows), 8)
    assert rel_l2(y.cpu().numpy()[:, rows], ref_o).max() < TIGHT


def test_wide_many_rows(dev):
    """600 000 rows (many workgroups per CU, each with its full tile count)."""
    K, N, T = 1664, 600000, 8
    gen = torch.Generator(device=dev)
    gen.manual_seed(7)
    nb = K // 128
    blk = torch.empty((N, nb, 28), dtype=torch.uint8, device=dev)
    blk[:, :, :24] = torch.randint(0, 243, (N, nb, 24), generator=gen, device=dev, dtype=torch.uint8)
    blk[:, :, 24:26] = torch.randint(0, 81, (N, nb, 2), generator=gen, device=dev, dtype=torch.uint8)
    blk[:, :, 26:28] = (torch.randn((N, nb), generator=gen, device=dev) * 0.02).abs().half() \
        .view(torch.uint8).view(N, nb, 2)
    W = blk.view(N, nb * 28)
    x_np = orc.synth_x(T, K, 3)
    y = ops.gemv_ptq1_wide(W, torch.from_numpy(x_np).to(dev), K, N).cpu().numpy()
    rows = np.concatenate([np.arange(0, N, 4999), np.arange(N - 200, N)])
    sub = W[torch.from_numpy(rows).to(dev)].cpu().numpy()
    ref = orc.gemv_ptq1(np.ascontiguousarray(sub), x_np.astype(np.float32), K, len(rows), T)
    assert rel_l2(y[:, rows], ref).max() < TIGHT


@pytest.mark.parametrize("K,Ns,T,dtype", [
    (5120, (17408, 17408), 8, np.float16),         # verifyWide's gate + up
    (5120, (10240, 6144), 5, np.float16),          # GDN qkv + z
    (5120, (12288, 1024, 1024), 3, np.float32),    # GQA q + k + v
    (1024, (37, 300, 5, 129), 8, np.float16),      # four ragged matrices, tiles across boundaries
    (6144, (5120, 5120), 2, np.float16),           # T = 2: the decode GEMV's batch form
])
def test_wide_batch_equals_single_calls(dev, K, Ns, T, dtype):
    """One batched launch equals the per-matrix calls bit for bit, and the oracle on sampled
    rows of every matrix."""
    Ws_np = [orc.synth_ptq1(N, K, K + N + i)[0] for i, N in enumerate(Ns)]
    x_np = orc.synth_x(T, K, K + T, dtype)
    Ws = [torch.from_numpy(w).to(dev) for w in Ws_np]
    x = torch.from_numpy(x_np).to(dev)
    ys = ops.gemv_ptq1_wide_batch(Ws, x, K, list(Ns))
    for W_np, W, N, y in zip(Ws_np, Ws, Ns, ys):
        assert torch.equal(y, ops.gemv_ptq1_wide(W, x, K, N)), N
        rows = np.unique(np.concatenate([np.arange(0, N, max(1, N // 53)), [N - 1]]))
        ref = orc.gemv_ptq1(np.ascontiguousarray(W_np[rows]), x_np.astype(np.float32), K, len(rows), T)
        assert rel_l2(y.cpu().numpy()[:, rows], ref).max() < TIGHT, N


def test_wide_nonfinite_tokens(dev):
    """A NaN or an infinity in a token's block makes that token's outputs NaN (as the
    reference's fp32 sum does) and leaves the other tokens exact."""
    K, N, T = 2048, 300, 4
    W_np, _, _ = orc.synth_ptq1(N, K, 11)
    x_np = orc.synth_x(T, K, 12)
    x_np[1, 200] = np.nan
    x_np[3, 1500] = np.inf
    W = torch.from_numpy(W_np).to(dev)
    y = ops.gemv_ptq1_wide(W, torch.from_numpy(x_np).to(dev), K, N).cpu().numpy()
    assert np.isnan(y[1]).all() and np.isnan(y[3]).all()
    ok = [0, 2]
    ref = orc.gemv_ptq1(W_np, x_np[ok].astype(np.float32), K, N, 2)
    assert rel_l2(y[ok], ref).max() < TIGHT
