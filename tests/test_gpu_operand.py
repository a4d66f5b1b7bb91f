"""The decode GEMV's operand form (KATA_XQ): the activation quantised once by its producer
(kata_gemv_prepare_x, or the input transforms with out_dtype KATA_XQ) instead of by every
workgroup of the GEMV.

Parity bar: bit-exact.  The GEMV on the operand form equals the GEMV on the raw rows bit
for bit (same quantiser, same operand bytes in LDS), and the raw-row GEMV is pinned to the
oracle by test_gpu_gemv.py; the transforms' operand form equals kata_gemv_prepare_x of their
own fp32 rows byte for byte.  The bytes themselves are decoded here by the documented
layout (A rows [m 2][g 4][2 t + limb][16 B] per block, quarter-major blocks, (s, 0) scale
pairs) and must give back x within the quantiser's bound amax / 65278 per element."""
import numpy as np
import pytest
import torch

from kata_amd import ops
from oracle import oracle as orc
from tests.conftest import rel_l2
from tests import operand_form
from tests.operand_form import decode as _decode

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("K,N,T,dtype,half2", [
    (128, 16, 1, np.float16, False), (384, 33, 2, np.float32, False), (1152, 40, 1, np.float32, False),
    (5120, 1000, 1, np.float16, False), (5120, 300, 2, np.float16, True), (6144, 129, 2, np.float32, False),
    (17408, 64, 1, np.float16, False), (17408, 40, 2, np.float16, False),
])
def test_operand_gemv_bit_exact(dev, K, N, T, dtype, half2):
    seed = K + 7 * N + T
    W_np, _, _ = orc.synth_ptq1(N, K, seed)
    x_np = orc.synth_x(T, K, seed + 1, dtype)
    W = torch.from_numpy(W_np).to(dev)
    x = torch.from_numpy(np.ascontiguousarray(x_np.T) if half2 else x_np).to(dev)
    xq = ops.gemv_prepare_x(x, K, T, half2=half2)
    assert xq.numel() == ops.gemv_xq_bytes(K, T)
    y_raw = ops.gemv_ptq1(W, x, K, N, T, half2=half2)
    y_xq = ops.gemv_ptq1(W, xq, K, N, T)
    assert torch.equal(y_raw, y_xq)
    ref = orc.gemv_ptq1(W_np, x_np.astype(np.float32), K, N, T)
    assert rel_l2(y_xq.cpu().numpy(), ref).max() < 2e-4
    # the bytes: x back within the block quantiser's bound (half a step of amax / 32639, plus
    # the fp32 rounding of x * 32639 / amax: a misplaced element is off by up to amax)
    xf = x_np.astype(np.float64)
    xd = _decode(xq.cpu().numpy(), K, T)
    amax = np.abs(xf.reshape(T, K // 128, 128)).max(axis=2)
    err = np.abs(xd - xf).reshape(T, K // 128, 128).max(axis=2)
    assert np.all(err <= amax / 65278 * 1.01 + 1e-30)


def test_operand_batch_and_nonfinite(dev):
    """The batch form on the operand form equals its raw-row launch; a block holding a NaN
    or an infinity gives NaN rows either way."""
    K, Ns, T = 5120, (700, 64, 9), 1
    mats = [orc.synth_ptq1(N, K, 90 + i)[0] for i, N in enumerate(Ns)]
    Ws = [torch.from_numpy(m).to(dev) for m in mats]
    x_np = orc.synth_x(T, K, 91, np.float32)
    for bad in (None, np.nan, np.inf):
        xb = x_np.copy()
        if bad is not None:
            xb[0, 3 * 128 + 5] = bad
        x = torch.from_numpy(xb).to(dev)
        xq = ops.gemv_prepare_x(x, K, T)
        for a, b in zip(ops.gemv_ptq1_batch(Ws, x, K, list(Ns), T), ops.gemv_ptq1_batch(Ws, xq, K, list(Ns), T)):
            assert torch.equal(a, b) or (bad is not None and torch.isnan(a).all() and torch.isnan(b).all())
            if bad is not None:
                assert torch.isnan(b).all()


def _signs(W, seed):
    return np.random.default_rng(seed).choice([-1.0, 1.0], size=W).astype(np.float32)


@pytest.mark.parametrize("M", [1, 2, 3, 8])
@pytest.mark.parametrize("mode,W", [(0, 5120), (1, 17408), (2, 6144), (3, 6144)])
def test_transform_writes_operand(dev, M, mode, W):
    """The transforms' operand form equals kata_gemv_prepare_x of their fp32 rows byte for
    byte (mode 0 through kata_add_rms_fwht with the residual add)."""
    rng = np.random.default_rng(10 * mode + M)
    t = lambda a: torch.from_numpy(a).to(dev)
    src = t(rng.standard_normal((M, W)).astype(np.float32))
    src2 = t(rng.standard_normal((M, W)).astype(np.float32))
    gs = t(_signs(W, mode))
    if mode == 0:
        f32, _, _ = ops.add_rms_fwht(src, gs, y=src2)
        xq, _, _ = ops.add_rms_fwht(src, gs, y=src2, out_dtype=torch.uint8)
    else:
        f32 = ops.rms_fwht(src, gs, mode, src2=src2 if mode == 1 else None)
        xq = ops.rms_fwht(src, gs, mode, src2=src2 if mode == 1 else None, out_dtype=torch.uint8)
    assert torch.equal(xq, ops.gemv_prepare_x(f32, W, M))


@pytest.mark.parametrize("K,Ns,T,dtype", [
    (384, (33,), 3, np.float32), (5120, (1000, 64), 4, np.float16), (5120, (300,), 8, np.float32),
    (17408, (40, 17), 5, np.float16), (6144, (129,), 7, np.float16),
])
def test_wide_operand_bit_exact(dev, K, Ns, T, dtype):
    """T = 3..8: the wide GEMV on the operand form (its prep kernel's image, written once)
    equals its launch on the raw rows bit for bit, single and batched; the bytes decode to x
    within the quantiser's bound, rows of tokens >= T zero."""
    seed = K + T
    mats = [orc.synth_ptq1(N, K, seed + i)[0] for i, N in enumerate(Ns)]
    Ws = [torch.from_numpy(m).to(dev) for m in mats]
    x_np = orc.synth_x(T, K, seed + 9, dtype)
    x = torch.from_numpy(x_np).to(dev)
    xq = ops.gemv_prepare_x(x, K, T)
    assert xq.numel() == K // 128 * 2080
    for W, N in zip(Ws, Ns):
        assert torch.equal(ops.gemv_ptq1_wide(W, x, K, N), ops.gemv_ptq1_wide(W, xq, K, N, T=T))
    for a, b in zip(ops.gemv_ptq1_wide_batch(Ws, x, K, list(Ns)), ops.gemv_ptq1_wide_batch(Ws, xq, K, list(Ns), T=T)):
        assert torch.equal(a, b)
    ref = orc.gemv_ptq1(mats[0], x_np.astype(np.float32), K, Ns[0], T)
    assert rel_l2(ops.gemv_ptq1_wide(Ws[0], xq, K, Ns[0], T=T).cpu().numpy(), ref).max() < 2e-4
    assert operand_form.bound_ok(operand_form.decode(xq.cpu().numpy(), K, T), x_np.astype(np.float64))
