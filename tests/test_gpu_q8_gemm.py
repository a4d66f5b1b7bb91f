"""GPU parity of the Q8_0 prefill GEMM (the MTP head's K/V catch-up: k_expand_q8 + dGemm,
src/engine.cpp:392-401, shaders/mtp.metal:24-33) against the CPU oracle.

Bars: the fused fp16 decode bit-exact (A = unit rows picks single weights, whose one fp32
product is exact); outputs within 1e-5 relative L2 per row of the oracle's double sums
(fp32 accumulation, fp16 operands as the reference's); fp16 outputs within 1e-3."""
import numpy as np
import pytest
import torch

from kata_amd import ops
from oracle import oracle as orc
from tests.conftest import rel_l2

pytestmark = pytest.mark.gpu


def _q8_extreme(N, K, seed):
    """Q8_0 bytes with scales whose products span fp16 subnormals to 2.6e4 (no overflow: a
    unit row times a row holding an infinity would sum 0 * inf)."""
    rng = np.random.default_rng(seed)
    q = rng.integers(-128, 128, size=(N, K), dtype=np.int64).astype(np.int8)
    mag = rng.choice([1e-7, 3e-5, 0.02, 1.0, 200.0], size=(N, K // 32))
    d = (mag * rng.choice([-1.0, 1.0], size=mag.shape)).astype(np.float16)
    return orc.q8_pack(q, d)


def test_q8_gemm_decode_bit_exact(dev):
    """C = I * Wexp^T with A the identity: every output is one weight half(d * q)."""
    K, N = 256, 96
    W_np = _q8_extreme(N, K, 5)
    A = torch.eye(K, dtype=torch.float16, device=dev)
    C = ops.gemm_q8_f16(A, torch.from_numpy(W_np).to(dev), K, N).cpu().numpy()      # [K][N]
    ref = orc.expand_q8_f16(W_np, K, N).astype(np.float32).T
    # equal values (a weight -0 sums to +0 with the zero products of the other columns)
    bad = C != ref
    assert not bad.any(), (int(bad.sum()), C[bad][:5], ref[bad][:5])


@pytest.mark.parametrize("M,K,N", [(7, 128, 48), (64, 1024, 200), (300, 2048, 130), (33, 5120, 1024)])
def test_q8_gemm_vs_oracle(dev, M, K, N):
    W_np, _, _ = orc.synth_q8(N, K, M + K + N)
    A_np = orc.synth_x(M, K, M + K + N + 1)
    W, A = torch.from_numpy(W_np).to(dev), torch.from_numpy(A_np).to(dev)
    C = ops.gemm_q8_f16(A, W, K, N).cpu().numpy()
    ref = orc.gemm_q8_f16(A_np, W_np, M, K, N)
    assert rel_l2(C, ref).max() < 1e-5
    C16 = ops.gemm_q8_f16(A, W, K, N, out_dtype=torch.float16).float().cpu().numpy()
    assert rel_l2(C16, ref).max() < 1e-3


@pytest.mark.parametrize("M,K,N", [(512, 10240, 5120), (512, 5120, 1024), (1000, 5120, 1024)])
def test_q8_gemm_mtp_shapes(dev, M, K, N):
    """The catch-up's shapes: eh_proj 10240 -> 5120, wk / wv 5120 -> 1024; the oracle on
    sampled weight rows, a torch fp32 product of the torch-expanded weights on all."""
    W_np, q, d = orc.synth_q8(N, K, K + N)
    A_np = orc.synth_x(M, K, K + N + 3)
    W, A = torch.from_numpy(W_np).to(dev), torch.from_numpy(A_np).to(dev)
    C = ops.gemm_q8_f16(A, W, K, N)
    wexp = (torch.from_numpy(q).to(dev).float().view(N, K // 32, 32) *
            torch.from_numpy(d.astype(np.float32)).to(dev)[:, :, None]).half().view(N, K)
    ref = A.float() @ wexp.float().T
    torch.cuda.synchronize()
    assert rel_l2(C.cpu().numpy(), ref.cpu().numpy()).max() < 1e-5
    rows = np.arange(0, N, 97)
    ref_o = orc.gemm_q8_f16(A_np[:64], np.ascontiguousarray(W_np[rows]), 64, K, len(rows))
    assert rel_l2(C.cpu().numpy()[:64, rows], ref_o).max() < 1e-5


def test_q8_gemm_strided_and_unaligned(dev):
    """lda > K, ldc > N through views, a weight base at a 4-byte (not 16-byte) offset."""
    M, K, N = 40, 1024, 72
    W_np, _, _ = orc.synth_q8(N, K, 3)
    buf = torch.zeros(W_np.size + 4, dtype=torch.uint8, device=dev)
    buf[4:] = torch.from_numpy(W_np.ravel()).to(dev)
    W = buf[4:]
    Abig = torch.from_numpy(orc.synth_x(M, K + 64, 4)).to(dev)
    out = torch.full((M, N + 8), 7.0, device=dev)
    ops.gemm_q8_f16(Abig, W, K, N, out=out)
    ref = orc.gemm_q8_f16(Abig.cpu().numpy()[:, :K], W_np, M, K, N)
    assert rel_l2(out.cpu().numpy()[:, :N], ref).max() < 1e-5
    assert (out.cpu().numpy()[:, N:] == 7.0).all()
