"""GPU parity at the full 27B shapes that bench.py times, and the activation contract.

References: the oracle (oracle/) on sampled rows, and a torch fp32 product of the weights
decoded on the GPU by the bit-exact expansion (PTQ1_0) or by torch from the block bytes
(Q8_0).  Bars: relative L2 <= 2e-4 per output vector for the 16-bit-activation GEMVs,
1e-5 for the Q8_0 GEMV (fp32 arithmetic), 5e-5 / 1e-5 for the fp16 / int8 prefill paths.

Activation contract of the PTQ1_0 GEMVs (quantised per 128-block to 16-bit fixed point,
s = amax / 32639): for every output row n,
    |y[n] - y_exact[n]| <= sum_b |d[n,b]| * nnz(trit[n,b,:]) * amax_b / 65000
                           + 4e-6 * sum_b |d[n,b]| * sum_e |trit[n,b,e] * x[128b + e]|,
the first term the worst case of the activation rounding (each element within half a
step s / 2 = amax / 65278, widened by the fp32 rounding of x / s and of s), the second the
fp32 accumulation.  Tested here with block outliers of 1e3 and 1e4
and with outlier channels, where it is far looser than 2e-4 relative L2 for the rows that
do not see the outlier; the per-vector relative L2 stays inside the 1e-3 contract.
A block holding a NaN or an infinity makes every output of that token NaN, as the
reference's coefficient-form sum does (its block `sumy` is then non-finite,
shaders/gemv_fast.metal:21-45).
"""
import numpy as np
import pytest
import torch

from kata_amd import ops
from oracle import oracle as orc
from tests.conftest import rel_l2

pytestmark = pytest.mark.gpu
TIGHT = 2e-4


def _exp(W, K, N):
    return ops.expand_f16(W, K, N).float()


@pytest.mark.parametrize("name,K,Ns", [("gdn_qkv_z", 5120, (10240, 6144)),
                                       ("attn_q_k_v", 5120, (12288, 1024, 1024)),
                                       ("ffn_gate_up", 5120, (17408, 17408))])
def test_batched_launch_full_shape(dev, name, K, Ns):
    """The batched launches bench.py times, at their full row counts, T = 1 and 2."""
    Ws_np = [orc.synth_ptq1(N, K, 300 + i + K)[0] for i, N in enumerate(Ns)]
    Ws = [torch.from_numpy(w).to(dev) for w in Ws_np]
    x_np = orc.synth_x(2, K, 301 + K)
    x = torch.from_numpy(x_np).to(dev)
    for T in (1, 2):
        xt = x[:T].contiguous()
        ys = ops.gemv_ptq1_batch(Ws, xt, K, list(Ns), T)
        for W, W_np, N, y in zip(Ws, Ws_np, Ns, ys):
            ref = xt.float() @ _exp(W, K, N).T
            torch.cuda.synchronize()
            err = rel_l2(y.cpu().numpy(), ref.cpu().numpy())
            assert err.max() < TIGHT, (name, T, N, err.max())
            rows = np.arange(0, N, 211)
            ref_o = orc.gemv_ptq1(np.ascontiguousarray(W_np[rows]), x_np[:T].astype(np.float32), K, len(rows), T)
            assert rel_l2(y.cpu().numpy()[:, rows], ref_o).max() < TIGHT
            y1 = ops.gemv_ptq1(W, xt, K, N, T)
            torch.cuda.synchronize()
            assert torch.equal(y, y1)               # one launch per matrix: same result


def _q8_decode(W: torch.Tensor, K: int, N: int) -> torch.Tensor:
    """fp32 weights of a Q8_0 matrix, decoded by torch from the block bytes."""
    blk = W.view(N, K // 32, 34)
    d = blk[:, :, 0:2].contiguous().view(torch.float16).float()          # [N][K/32][1]
    q = blk[:, :, 2:].contiguous().view(torch.int8).float()              # [N][K/32][32]
    return (q * d).reshape(N, K)


@pytest.mark.parametrize("K,N", [(5120, 17408), (17408, 5120)])
def test_q8_full_shape(dev, K, N):
    """BASELINE config 3 Q8_0 MTP-head shapes, T = 1 and 2."""
    W_np, _, _ = orc.synth_q8(N, K, 400 + K)
    W = torch.from_numpy(W_np).to(dev)
    x_np = orc.synth_x(2, K, 401 + K)
    x = torch.from_numpy(x_np).to(dev)
    Wf = _q8_decode(W, K, N)
    for T in (1, 2):
        y = ops.gemv_q8(W, x[:T].contiguous(), K, N, T)
        ref = x[:T].float() @ Wf.T
        torch.cuda.synchronize()
        assert rel_l2(y.cpu().numpy(), ref.cpu().numpy()).max() < 1e-5
        rows = np.arange(0, N, 173)
        ref_o = orc.gemv_q8(np.ascontiguousarray(W_np[rows]), x_np[:T].astype(np.float32), K, len(rows), T)
        assert rel_l2(y.cpu().numpy()[:, rows], ref_o).max() < 1e-5


def test_prefill_m7300_down_shape(dev):
    """BASELINE config 5 prefill, the down projection (17408 -> 5120) at M = 7300, on the fp16
    exact path and on the int8 path (the gate shape is in test_gpu_q8_prefill.py)."""
    M, K, N = 7300, 17408, 5120
    W_np, _, _ = orc.synth_ptq1(N, K, 5105)
    W = torch.from_numpy(W_np).to(dev)
    A = torch.from_numpy(orc.synth_x(M, K, 5106)).to(dev)
    C = ops.gemm_ptq1_f16(A, W, K, N)
    ref = A.float() @ _exp(W, K, N).T
    assert rel_l2(C.cpu().numpy(), ref.cpu().numpy()).max() < 5e-5
    del ref, C
    Q, SX = ops.quant_rows(A)
    C8 = ops.gemm_ptq1_i8(Q, SX, W, K, N)
    T8, SW = ops.expand_i8(W, K, N)
    ref8 = torch.zeros((M, N), dtype=torch.float32, device=dev)
    for g in range(K // 128):
        I = Q[:, 128 * g:128 * (g + 1)].float() @ T8[:, 128 * g:128 * (g + 1)].float().T
        ref8 += I * (SW[:, g][None, :] * SX[g, :M][:, None])
    assert rel_l2(C8.cpu().numpy(), ref8.cpu().numpy()).max() < 1e-5


def _contract_bound(trits, scales, x):
    """Per-row worst case of the 16-bit block activation rounding (see the module doc)."""
    N, K = trits.shape
    nb = K // 128
    amax = np.abs(x.astype(np.float64)).reshape(nb, 128).max(-1)                  # [nb]
    nnz = (trits != 0).reshape(N, nb, 128).sum(-1).astype(np.float64)             # [N][nb]
    d = np.abs(scales.astype(np.float64))                                         # [N][nb]
    return (d * nnz * (amax / 65000.0)[None, :]).sum(-1)


@pytest.mark.parametrize("case", ["block1e3", "block1e4", "channels1e4"])
def test_outlier_activations_full_shape(dev, case):
    K, N = 5120, 17408
    W_np, trits, scales = orc.synth_ptq1(N, K, 2100)
    W = torch.from_numpy(W_np).to(dev)
    x = orc.synth_x(1, K, 2101, np.float32)
    if case == "block1e3":
        x[0, 7::128] *= 1e3                     # one element of every block 1000x its peers
    elif case == "block1e4":
        x[0, 7::128] *= 1e4
    else:
        x[0, [100, 2000, 4097]] = [3e4, -2e4, 1.5e4]   # a few huge channels
    y = ops.gemv_ptq1(W, torch.from_numpy(x).to(dev), K, N, 1)
    Wexp = _exp(W, K, N).double()
    xd = torch.from_numpy(x).to(dev).double()
    ref = (xd @ Wexp.T)[0]
    sum_abs = (xd.abs() @ Wexp.abs().T)[0]
    torch.cuda.synchronize()
    err = np.abs(y.cpu().numpy()[0].astype(np.float64) - ref.cpu().numpy())
    bound = _contract_bound(trits, scales, x[0]) + 4e-6 * sum_abs.cpu().numpy()
    assert (err <= bound).all(), (case, float((err / bound).max()))
    r = rel_l2(y.cpu().numpy(), ref.cpu().numpy()[None]).max()
    print(f"{case}: rel L2 {r:.2e}, worst err/bound {(err / bound).max():.3f}")
    assert r < 1e-3


@pytest.mark.parametrize("bad", [float("nan"), float("inf"), float("-inf")])
def test_non_finite_activation_propagates(dev, bad):
    K, N = 1024, 96
    W_np, _, _ = orc.synth_ptq1(N, K, 77)
    W = torch.from_numpy(W_np).to(dev)
    for dt in (torch.float32, torch.float16):
        x = torch.from_numpy(orc.synth_x(8, K, 78, np.float32)).to(dev)
        x[0, 300] = bad                              # token 0 only
        x = x.to(dt)
        y1 = ops.gemv_ptq1(W, x[:1].contiguous(), K, N, 1)
        y2 = ops.gemv_ptq1(W, x[:2].contiguous(), K, N, 2)
        yw = ops.gemv_ptq1_wide(W, x, K, N)          # T = 8: the wide kernel
        torch.cuda.synchronize()
        for y in (y1, y2, yw):
            assert torch.isnan(y[0]).all()
            assert torch.isfinite(y[1:]).all()
