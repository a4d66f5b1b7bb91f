"""The Q8_0 GEMV's batch form (the MTP block's wq + wk + wv and gate + up in one launch each,
src/engine.cpp:361,369) and its dispatcher entry: every matrix of a batch equals its single
launch bit for bit and the oracle within the single launch's bar (1e-5 relative L2 per
output vector), at ragged and at the MTP head's full shapes, for T = 1 and 2 and both
activation dtypes."""
import numpy as np
import pytest
import torch

from kata_amd import ops
from kata_amd.engine import Dispatch
from oracle import oracle as orc
from tests.conftest import rel_l2

pytestmark = pytest.mark.gpu


def _mats(K, Ns, seed, shift=0):
    """Q8_0 matrices; `shift` bytes of padding before each puts the blocks at 2-byte alignment."""
    out = []
    for i, N in enumerate(Ns):
        W_np, _, _ = orc.synth_q8(N, K, seed + 13 * i)
        buf = torch.zeros(W_np.size + 16, dtype=torch.uint8)
        buf[shift:shift + W_np.size] = torch.from_numpy(W_np.ravel())
        out.append((W_np, buf))
    return out


@pytest.mark.parametrize("K,Ns,T,dtype,shift", [
    (256, (37, 5), 1, np.float16, 0),
    (5120, (1000, 129, 7, 64), 1, np.float32, 2),
    (5120, (300, 64, 64), 2, np.float16, 2),
    (17408, (24, 40), 2, np.float32, 0),
    (10240, (8, 3, 16), 1, np.float16, 0),
])
def test_batch_equals_single_and_oracle(dev, K, Ns, T, dtype, shift):
    mats = _mats(K, Ns, K + T, shift)
    x = torch.from_numpy(orc.synth_x(T, K, K + 5, dtype)).to(dev)
    Ws = [buf.to(dev)[shift:shift + W_np.size] for W_np, buf in mats]
    ys = ops.gemv_q8_batch(Ws, x, K, list(Ns), T)
    for (W_np, _), W, y, N in zip(mats, Ws, ys, Ns):
        single = ops.gemv_q8(W, x, K, N, T)
        assert torch.equal(y, single), N
        ref = orc.gemv_q8(W_np, x.cpu().numpy().astype(np.float32), K, N, T)
        assert rel_l2(y.cpu().numpy(), ref).max() < 1e-5, N


@pytest.mark.parametrize("T", [1, 2])
def test_mtp_shapes_full(dev, T):
    """wq + wk + wv (5120 -> 12288, 1024, 1024) and gate + up (5120 -> 17408 each), full
    rows, against single launches bit for bit and the oracle on sampled rows."""
    K = 5120
    for Ns, seed in (((12288, 1024, 1024), 70), ((17408, 17408), 80)):
        mats = [orc.synth_q8(N, K, seed + i)[0] for i, N in enumerate(Ns)]
        Ws = [torch.from_numpy(m).to(dev) for m in mats]
        x = torch.from_numpy(orc.synth_x(T, K, seed + 9, np.float16)).to(dev)
        ys = ops.gemv_q8_batch(Ws, x, K, list(Ns), T)
        for W_np, W, y, N in zip(mats, Ws, ys, Ns):
            assert torch.equal(y, ops.gemv_q8(W, x, K, N, T))
            rows = np.random.default_rng(seed).choice(N, 96, replace=False)
            sub = W_np.reshape(N, -1)[rows]
            ref = orc.gemv_q8(sub, x.cpu().numpy().astype(np.float32), K, len(rows), T)
            assert rel_l2(y.cpu().numpy()[:, rows], ref).max() < 1e-5


def test_dispatch_gemv_q8_offsets(dev):
    """The dispatcher's `gq`: matrices at byte offsets of one weight buffer (the second at a
    2-byte-aligned offset, as Q8_0 tensors can sit in a GGUF data region)."""
    K, Ns = 2048, (96, 40, 40)
    mats = [orc.synth_q8(N, K, 90 + i)[0] for i, N in enumerate(Ns)]
    parts, offs, o = [], [], 0
    for m in mats:
        pad = 2 if o % 4 == 0 else 0
        parts.append(np.zeros(pad, np.uint8))
        o += pad
        offs.append(o)
        parts.append(m.ravel())
        o += m.size
    buf = torch.from_numpy(np.concatenate(parts)).to(dev)
    d = Dispatch(buf)
    for T in (1, 2):
        x = torch.from_numpy(orc.synth_x(T, K, 99 + T, np.float32)).to(dev)
        outs = [torch.empty((T, N), device=dev) for N in Ns]
        d.gemv_q8(offs, x, outs, K, list(Ns))
        for m, y, N in zip(mats, outs, Ns):
            ref = orc.gemv_q8(m, x.cpu().numpy(), K, N, T)
            assert rel_l2(y.cpu().numpy(), ref).max() < 1e-5
