"""GPU parity of the Q8_0 GEMV, the PTQ1_0 expansions, the fused fp16 prefill GEMM and
the int8 prefill path against the CPU oracle.

Bars: decoded trits / fp16 weights / int8 codes / int32 group sums bit-exact;
fp32-accumulated outputs within 1e-3 relative L2 per output vector (tighter where the
arithmetic allows)."""
import numpy as np
import pytest
import torch

from kata_amd import ops
from kata_amd.engine import Dispatch
from oracle import oracle as orc
from tests.conftest import rel_l2

pytestmark = pytest.mark.gpu


# ----------------------------------------------------------------------------- Q8_0
def test_q8_golden(dev, golden):
    W = torch.from_numpy(golden["q8_W"]).to(dev)
    x = torch.from_numpy(golden["q8_x"]).to(dev)
    y = ops.gemv_q8(W, x, 64, 8, 2).cpu().numpy()
    assert rel_l2(y, golden["q8_y"]).max() < 1e-5


@pytest.mark.parametrize("K,N,T,dtype", [
    (64, 1, 1, np.float32), (96, 7, 2, np.float16),       # odd block count: one-block tail
    (32, 5, 1, np.float16), (8224, 9, 1, np.float16),     # one block; odd count, sliced rows
    (8224, 6, 2, np.float32),
    (5120, 40, 1, np.float16), (5120, 33, 2, np.float32),
    (17408, 24, 2, np.float16), (10240, 16, 1, np.float32),
])
def test_q8_random(dev, K, N, T, dtype):
    W_np, _, _ = orc.synth_q8(N, K, K + N)
    x_np = orc.synth_x(T, K, K + N + 1, dtype)
    y = ops.gemv_q8(torch.from_numpy(W_np).to(dev), torch.from_numpy(x_np).to(dev), K, N, T).cpu().numpy()
    ref = orc.gemv_q8(W_np, x_np.astype(np.float32), K, N, T)
    assert rel_l2(y, ref).max() < 1e-5


@pytest.mark.parametrize("K,N,T", [(64, 5, 1), (8192, 9, 2), (96, 3, 1), (8224, 5, 1), (32, 3, 2)])
def test_q8_unaligned_weight_base(dev, K, N, T):
    """Weights at a 2-byte (not 4-byte) aligned address: every block changes alignment."""
    W_np, _, _ = orc.synth_q8(N, K, 7 * K + N)
    buf = torch.zeros(W_np.size + 16, dtype=torch.uint8, device=dev)
    W = buf[2:2 + W_np.size]
    W.copy_(torch.from_numpy(W_np.reshape(-1)))
    assert W.data_ptr() % 4 == 2
    x_np = orc.synth_x(T, K, K + 3, np.float16)
    y = ops.gemv_q8(W, torch.from_numpy(x_np).to(dev), K, N, T).cpu().numpy()
    ref = orc.gemv_q8(W_np, x_np.astype(np.float32), K, N, T)
    assert rel_l2(y, ref).max() < 1e-5


# ----------------------------------------------------------------------------- expansions
def test_expand_bit_exact(dev, golden):
    K, N = int(golden["ptq1_K"]), int(golden["ptq1_N"])
    W = torch.from_numpy(golden["ptq1_W"]).to(dev)
    e = ops.expand_f16(W, K, N).cpu().numpy()
    assert np.array_equal(e.view(np.uint16), golden["expand_f16"].view(np.uint16))
    T8, SW = ops.expand_i8(W, K, N)
    assert np.array_equal(T8.cpu().numpy(), golden["ptq1_trits"])
    assert np.array_equal(SW.cpu().numpy(), golden["ptq1_scales"].astype(np.float32))


def test_expand_random_bytes_bit_exact(dev):
    # arbitrary bytes (incl. 243..255, never produced by the quantiser) decode like the oracle
    rng = np.random.default_rng(11)
    N, K = 64, 1024
    W_np = rng.integers(0, 256, (N, K // 128 * 28), dtype=np.uint8)
    W_np.reshape(N, K // 128, 28)[:, :, 26:28] = np.array([0.375], np.float16).view(np.uint8)  # finite scales
    W = torch.from_numpy(W_np).to(dev)
    e = ops.expand_f16(W, K, N).cpu().numpy()
    assert np.array_equal(e.view(np.uint16), orc.expand_f16(W_np, K, N).view(np.uint16))
    T8, _ = ops.expand_i8(W, K, N)
    assert np.array_equal(T8.cpu().numpy(), orc.expand_i8(W_np, K, N)[0])


# ----------------------------------------------------------------------------- fp16 GEMM
def test_gemm_f16_golden(dev, golden):
    K, N = int(golden["ptq1_K"]), int(golden["ptq1_N"])
    A = torch.from_numpy(golden["gemm_A"]).to(dev)
    W = torch.from_numpy(golden["ptq1_W"]).to(dev)
    C = ops.gemm_ptq1_f16(A, W, K, N).cpu().numpy()
    assert rel_l2(C, golden["gemm_C"]).max() < 1e-5


@pytest.mark.parametrize("M,K,N", [(1, 128, 16), (5, 384, 130), (130, 1024, 64), (257, 640, 300)])
def test_gemm_f16_random(dev, M, K, N):
    W_np, _, _ = orc.synth_ptq1(N, K, M + K + N)
    A_np = orc.synth_x(M, K, M + 1)
    C = ops.gemm_ptq1_f16(torch.from_numpy(A_np).to(dev), torch.from_numpy(W_np).to(dev), K, N).cpu().numpy()
    ref = orc.gemm_f16(A_np, W_np, M, K, N)
    assert rel_l2(C, ref).max() < 1e-5


@pytest.mark.parametrize("K,N", [(5120, 17408), (17408, 5120)])
def test_gemm_f16_pp512_full_shape(dev, K, N):
    """BASELINE config 4 shapes: every row vs torch fp32 on the bit-exact expanded weights,
    plus oracle rows; fp16 output within fp16 rounding of the fp32 output."""
    M = 512
    W_np, _, _ = orc.synth_ptq1(N, K, K ^ N)
    A_np = orc.synth_x(M, K, 99)
    A = torch.from_numpy(A_np).to(dev)
    W = torch.from_numpy(W_np).to(dev)
    C = ops.gemm_ptq1_f16(A, W, K, N)
    ref = A.float() @ ops.expand_f16(W, K, N).float().T
    # both sides accumulate in fp32 in different orders: ~eps*sqrt(K) apart
    assert rel_l2(C.cpu().numpy(), ref.cpu().numpy()).max() < 5e-5
    Ch = ops.gemm_ptq1_f16(A, W, K, N, out_dtype=torch.float16)
    assert torch.equal(Ch, C.half())
    rows = [0, 1, 255, 511]
    ref_o = orc.gemm_f16(np.ascontiguousarray(A_np[rows]), W_np[:64], len(rows), K, 64)
    assert rel_l2(C.cpu().numpy()[rows, :64], ref_o).max() < 1e-5


def test_gemm_f16_tile_schedules(dev):
    """Whole-tile rounds, split tiles (pieces summed from the workspace) and both together,
    called back to back so the workspace is reused with a different piece count; every
    output vs torch fp32 on the bit-exact expanded weights."""
    cases = [(256, 128, 128 * 256),      # 256 tiles: whole tiles only (one round on 256 CUs)
             (256, 256, 128 * 257 - 5),  # one round + 1 split tile of 2 pieces, ragged N
             (70, 1280, 200),            # 2 tiles split 10 ways
             (513, 384, 130)]            # 3 x 2 tiles, 3 pieces, ragged M and N
    for M, K, N in cases:
        W_np, _, _ = orc.synth_ptq1(N, K, M * 7 + K + N)
        A = torch.from_numpy(orc.synth_x(M, K, M + 3)).to(dev)
        W = torch.from_numpy(W_np).to(dev)
        C = ops.gemm_ptq1_f16(A, W, K, N)
        ref = A.float() @ ops.expand_f16(W, K, N).float().T
        assert rel_l2(C.cpu().numpy(), ref.cpu().numpy()).max() < 5e-5, (M, K, N)


@pytest.mark.parametrize("M", [1024, 7300])
def test_gemm_config5_prefill_shapes(dev, M):
    """BASELINE config 5 prefill: a 7300-token prompt as one GEMM and as the reference's
    1024-row chunk, gate shape, on the fp16 exact path and on the int8 FFN path.  References:
    torch fp32 on the bit-exact expanded weights; for int8 the per-group integer sums come
    from fp32 matmuls of integer values (exact below 2^24) and fold in ascending group order."""
    K, N = 5120, 17408
    W_np, _, _ = orc.synth_ptq1(N, K, 5005)
    W = torch.from_numpy(W_np).to(dev)
    A = torch.from_numpy(orc.synth_x(M, K, 5006)).to(dev)
    C = ops.gemm_ptq1_f16(A, W, K, N)
    ref = A.float() @ ops.expand_f16(W, K, N).float().T
    assert rel_l2(C.cpu().numpy(), ref.cpu().numpy()).max() < 5e-5
    del ref
    Q, SX = ops.quant_rows(A)
    C8 = ops.gemm_ptq1_i8(Q, SX, W, K, N)
    T8, SW = ops.expand_i8(W, K, N)
    ref8 = torch.zeros((M, N), dtype=torch.float32, device=dev)
    for g in range(K // 128):
        I = Q[:, 128 * g:128 * (g + 1)].float() @ T8[:, 128 * g:128 * (g + 1)].float().T
        ref8 += I * (SW[:, g][None, :] * SX[g, :M][:, None])
    assert rel_l2(C8.cpu().numpy(), ref8.cpu().numpy()).max() < 1e-5


# ----------------------------------------------------------------------------- int8 path
def test_quant_rows_bit_exact(dev, golden):
    Q, SX = ops.quant_rows(torch.from_numpy(golden["qr_X"]).to(dev))
    assert np.array_equal(Q.cpu().numpy(), golden["qr_Q"])
    assert np.array_equal(SX.cpu().numpy().view(np.uint32), golden["qr_SX"].view(np.uint32))
    X = orc.synth_x(37, 5120, 12)
    X[3, 128:256] = 0
    Q, SX = ops.quant_rows(torch.from_numpy(X).to(dev), ldS=64)
    Qo, SXo = orc.quant_rows(X, 37, 5120, 64)
    assert np.array_equal(Q.cpu().numpy(), Qo)
    assert np.array_equal(SX.cpu().numpy()[:, :37].view(np.uint32), SXo[:, :37].view(np.uint32))


def test_gemm_i8_integer_sums_exact(dev):
    """Unit scales: C equals the exact integer sum (< 2^24), whatever the order."""
    rng = np.random.default_rng(13)
    M, K, N = 70, 1024, 96
    t = rng.integers(-1, 2, (N, K)).astype(np.int8)
    W_np = orc.pack(t, np.ones((N, K // 128), np.float16))
    A8 = rng.integers(-127, 128, (M, K)).astype(np.int8)
    SX = np.ones((K // 128, M), np.float32)
    C = ops.gemm_ptq1_i8(torch.from_numpy(A8).to(dev), torch.from_numpy(SX).to(dev),
                         torch.from_numpy(W_np).to(dev), K, N).cpu().numpy()
    want = A8.astype(np.int64) @ t.astype(np.int64).T
    assert np.array_equal(C.astype(np.int64), want)


def test_gemm_i8_golden_and_random(dev, golden):
    K, N = int(golden["ptq1_K"]), int(golden["ptq1_N"])
    C = ops.gemm_ptq1_i8(torch.from_numpy(golden["qr_Q"]).to(dev), torch.from_numpy(golden["qr_SX"]).to(dev),
                         torch.from_numpy(golden["ptq1_W"]).to(dev), K, N).cpu().numpy()
    ref = orc.gemm_i8(golden["qr_Q"], golden["qr_SX"], golden["ptq1_W"], 3, K, N)
    assert rel_l2(C, ref).max() < 1e-6
    M, K, N = 200, 5120, 160
    W_np, _, _ = orc.synth_ptq1(N, K, 14)
    X = orc.synth_x(M, K, 15)
    Q, SX = orc.quant_rows(X, M, K)
    Cg = ops.gemm_ptq1_i8(torch.from_numpy(Q).to(dev), torch.from_numpy(SX).to(dev),
                          torch.from_numpy(W_np).to(dev), K, N).cpu().numpy()
    assert rel_l2(Cg, orc.gemm_i8(Q, SX, W_np, M, K, N)).max() < 1e-6


@pytest.mark.parametrize("M,K,N", [(1, 128, 1), (1, 128, 129), (3, 256, 5), (257, 128, 130), (300, 384, 257)])
def test_gemm_i8_edge_shapes(dev, M, K, N):
    """int8 GEMM at edge shapes: one token row, one 128-group (a single stage), one output
    column, ragged row and column tiles, and a scale row stride wider than M (ldS = M + 7),
    with fp32 and fp16 outputs; vs the oracle's int8 path on the same Q and SX."""
    W_np, _, _ = orc.synth_ptq1(N, K, M * 31 + K + N)
    Q, SX = orc.quant_rows(orc.synth_x(M, K, M + 77), M, K, M + 7)
    ref = orc.gemm_i8(Q, SX, W_np, M, K, N)
    args = (torch.from_numpy(Q).to(dev), torch.from_numpy(SX).to(dev), torch.from_numpy(W_np).to(dev), K, N)
    C = ops.gemm_ptq1_i8(*args).cpu().numpy()
    assert rel_l2(C, ref).max() < 1e-6, (M, K, N)
    C16 = ops.gemm_ptq1_i8(*args, out_dtype=torch.float16).cpu().numpy().astype(np.float32)
    assert rel_l2(C16, ref).max() < 1e-3, (M, K, N)        # fp16 rounding: <= 2^-11 per element


def test_gemm_i8_pp512_and_tail_tiles(dev):
    """Shapes just past one round of whole tiles (M = 512, 16384 < N: 256 whole tiles and a
    tail split into K pieces): a ragged case (300 x 256 x 17000) vs the oracle, and the pp512
    gate shape vs per-group fp32 matmuls (exact integer sums) folded in ascending group order."""
    M, K, N = 300, 256, 17000
    W_np, _, _ = orc.synth_ptq1(N, K, 4401)
    Q, SX = orc.quant_rows(orc.synth_x(M, K, 4402), M, K)
    C = ops.gemm_ptq1_i8(torch.from_numpy(Q).to(dev), torch.from_numpy(SX).to(dev),
                         torch.from_numpy(W_np).to(dev), K, N).cpu().numpy()
    assert rel_l2(C, orc.gemm_i8(Q, SX, W_np, M, K, N)).max() < 1e-6
    M, K, N = 512, 5120, 17408
    W = torch.from_numpy(orc.synth_ptq1(N, K, 4403)[0]).to(dev)
    A = torch.from_numpy(orc.synth_x(M, K, 4404)).to(dev)
    Q, SX = ops.quant_rows(A)
    C8 = ops.gemm_ptq1_i8(Q, SX, W, K, N)
    T8, SW = ops.expand_i8(W, K, N)
    ref8 = torch.zeros((M, N), dtype=torch.float32, device=dev)
    for g in range(K // 128):
        I = Q[:, 128 * g:128 * (g + 1)].float() @ T8[:, 128 * g:128 * (g + 1)].float().T
        ref8 += I * (SW[:, g][None, :] * SX[g, :M][:, None])
    assert rel_l2(C8.cpu().numpy(), ref8.cpu().numpy()).max() < 1e-5


# ----------------------------------------------------------------------------- dispatcher
def test_gemm_i8_tile_schedules(dev):
    """int8 GEMM over whole tiles plus K-pieces (513 tiles of 256x128 on 256 slots) and
    pieces only, back to back; vs the oracle's int8 path."""
    for M, K, N in ((128, 256, 128 * 513 - 7), (200, 1280, 300)):
        W_np, _, _ = orc.synth_ptq1(N, K, M + K + N + 5)
        A = torch.from_numpy(orc.synth_x(M, K, M + 9)).to(dev)
        Q, SX = ops.quant_rows(A)
        C = ops.gemm_ptq1_i8(Q, SX, torch.from_numpy(W_np).to(dev), K, N).cpu().numpy()
        ref = orc.gemm_i8(Q.cpu().numpy(), SX.cpu().numpy(), W_np, M, K, N)
        assert rel_l2(C, ref).max() < 1e-6, (M, K, N)


def test_dispatch_offsets_and_i8_selection(dev):
    K, N = 1024, 64
    W1, _, _ = orc.synth_ptq1(N, K, 21)
    W2, _, _ = orc.synth_ptq1(N, K, 22)
    buf = torch.from_numpy(np.concatenate([W1.ravel(), W2.ravel()])).to(dev)
    d = Dispatch(buf)
    off2 = W1.size
    x = torch.from_numpy(orc.synth_x(1, K, 23, np.float32)).to(dev)
    y = torch.empty((1, N), dtype=torch.float32, device=dev)
    d.gemv(off2, x, y, K, N)
    assert rel_l2(y.cpu().numpy(), orc.gemv_ptq1(W2, x.cpu().numpy(), K, N, 1)).max() < 2e-4
    M = 48
    A = torch.from_numpy(orc.synth_x(M, K, 24)).to(dev)
    C = torch.empty((M, N), dtype=torch.float32, device=dev)
    d.set_i8("ffn")
    A8 = torch.empty((M, K), dtype=torch.int8, device=dev)
    SX = torch.empty((K // 128, M), dtype=torch.float32, device=dev)
    d.prefill(off2, A, C, K, N, "gate", A8, SX)          # int8 path
    Q, SXo = orc.quant_rows(A.cpu().numpy(), M, K)
    assert np.array_equal(A8.cpu().numpy(), Q)
    assert rel_l2(C.cpu().numpy(), orc.gemm_i8(Q, SXo, W2, M, K, N)).max() < 1e-6
    d.prefill(off2, A, C, K, N, "down")                  # fp16 exact path
    assert rel_l2(C.cpu().numpy(), orc.gemm_f16(A.cpu().numpy(), W2, M, K, N)).max() < 1e-5
