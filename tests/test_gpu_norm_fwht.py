"""GPU parity of the matmul input transform (residual add + RMSNorm / SwiGLU / GDN order,
sign, 1024-block Walsh-Hadamard) against the double-precision oracle."""
import numpy as np
import pytest
import torch

from kata_amd import ops
from oracle import oracle as orc

from conftest import rel_l2

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    return torch.device("cuda:0")


def _signs(W, seed, gamma=False):
    rng = np.random.default_rng(seed)
    s = rng.choice([-1.0, 1.0], size=W).astype(np.float32)
    if gamma:
        s *= (1.0 + 0.1 * rng.standard_normal(W)).astype(np.float32)
    return s


@pytest.mark.parametrize("M,add,want_h,out_dtype", [(1, True, True, torch.float32), (1, False, False, torch.float32),
                                                    (3, True, False, torch.float16), (300, True, True, torch.float16)])
def test_add_rms_fwht(dev, M, add, want_h, out_dtype):
    W = 5120
    rng = np.random.default_rng(M * 10 + add)
    x = rng.standard_normal((M, W)).astype(np.float32)
    y = rng.standard_normal((M, W)).astype(np.float32)
    gs, gamma = _signs(W, 1, gamma=True), (1.0 + 0.1 * rng.standard_normal(W)).astype(np.float32)
    t = lambda a: torch.from_numpy(a).to(dev)
    hd = torch.float16 if out_dtype == torch.float16 else torch.float32
    out, xnew, hout = ops.add_rms_fwht(t(x), t(gs), y=t(y) if add else None, gamma=t(gamma) if want_h else None,
                                       out_dtype=out_dtype, want_xnew=True, hout_dtype=hd)
    ref, href = orc.norm_fwht(x, gs, 0, src2=y if add else None, gamma=gamma if want_h else None, add=add)
    tol = 1e-3 if out_dtype == torch.float16 else 1e-5
    assert rel_l2(out.float().cpu().numpy(), ref).max() < tol
    assert np.array_equal(xnew.cpu().numpy(), x + y if add else x)
    if want_h:
        assert rel_l2(hout.float().cpu().numpy(), href).max() < tol


def test_add_rms_fwht_half2_verify_layout(dev):
    """M = 2 into the [W][2] half2 operand equals the two fp16 rows interleaved."""
    W = 5120
    rng = np.random.default_rng(9)
    x = torch.from_numpy(rng.standard_normal((2, W)).astype(np.float32)).to(dev)
    gs = torch.from_numpy(_signs(W, 2)).to(dev)
    rows, _, _ = ops.add_rms_fwht(x, gs, out_dtype=torch.float16)
    h2, _, _ = ops.add_rms_fwht(x, gs, half2=True)
    assert torch.equal(h2, rows.T.contiguous())


@pytest.mark.parametrize("mode,W,M", [(0, 5120, 4), (1, 17408, 4), (2, 6144, 4), (3, 6144, 4),
                                      (0, 5120, 64), (1, 5120, 70), (3, 5120, 64)])
def test_rms_fwht_modes(dev, mode, W, M):
    """Few rows take one workgroup per 1024-block, >= 64 rows of width 5120 one per row."""
    rng = np.random.default_rng(mode + 20)
    a = rng.standard_normal((M, W)).astype(np.float32)
    b = rng.standard_normal((M, W)).astype(np.float32)
    gs = _signs(W, 3 + mode)
    t = lambda v: torch.from_numpy(v).to(dev)
    out = ops.rms_fwht(t(a), t(gs), mode, src2=t(b) if mode == 1 else None)
    ref, _ = orc.norm_fwht(a, gs, mode, src2=b if mode == 1 else None)
    assert rel_l2(out.cpu().numpy(), ref).max() < 1e-5
    out16 = ops.rms_fwht(t(a), t(gs), mode, src2=t(b) if mode == 1 else None, out_dtype=torch.float16)
    assert rel_l2(out16.float().cpu().numpy(), ref).max() < 1e-3


def test_transform_feeds_the_gemv(dev):
    """The transform's fp16 output is a valid GEMV activation: y = W H(norm(x)) matches the
    oracle GEMV on the oracle's transform (end-to-end input path of one projection)."""
    K, N = 5120, 256
    rng = np.random.default_rng(31)
    x = rng.standard_normal((1, K)).astype(np.float32)
    gs = _signs(K, 4, gamma=True)
    W_np, _, _ = orc.synth_ptq1(N, K, 32)
    h, _, _ = ops.add_rms_fwht(torch.from_numpy(x).to(dev), torch.from_numpy(gs).to(dev), out_dtype=torch.float16)
    y = ops.gemv_ptq1(torch.from_numpy(W_np).to(dev), h, K, N, 1).cpu().numpy()
    ref_h, _ = orc.norm_fwht(x, gs, 0)
    ref = orc.gemv_ptq1(W_np, ref_h.astype(np.float32), K, N, 1)
    assert rel_l2(y, ref).max() < 2e-3
