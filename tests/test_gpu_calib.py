"""The measurement kernels behind the bench's calibration figures run cleanly on the GPU:
the empty kernel, the plain streaming read at every geometry of its sweep (including a size
that is not a whole number of 1 KB pieces), the read ceiling, and the decode GEMV's
weight-load stream alone in its run order, its tile-strided order and with padded blocks.
Each reads only inside its buffer and leaves the sentinel word alone (it is written only
when the fold of what was read hits one 32-bit value, which these inputs do not)."""
import pytest
import torch

from kata_amd import ops

pytestmark = pytest.mark.gpu


def _word(dev):
    return torch.zeros(4, dtype=torch.int32, device=dev)


def test_empty_and_plain_reads(dev):
    w = _word(dev)
    buf = torch.full((3 * 1024 * 1024 + 333,), 7, dtype=torch.uint8, device=dev)
    ops.calib_empty(w)
    ops.calib_read(buf, w)
    ops.calib_read(buf, w, nbytes=4096 + 16)
    ops.calib_read_peak(buf, w)
    for threads in (256, 512, 1024):
        for inflight in (2, 4, 8, 16):
            for nt in (False, True):
                ops.calib_read_cfg(buf, w, threads, 300, inflight, nt)
    torch.cuda.synchronize()
    assert torch.count_nonzero(w).item() == 0


@pytest.mark.parametrize("K,N", [(5120, 66000), (4096, 66000), (5120, 17408), (640, 1001), (17408, 37)])
def test_weight_stream(dev, K, N):
    """(5120, 66000): tile-strided order with a wave left idle; (4096, 66000): strided with
    all 16 waves; (5120, 17408): run order; (640, 1001): padded blocks, ragged rows;
    (17408, 37): fewer tiles than workgroups."""
    w = _word(dev)
    W = torch.full((N * (K // 128) * 28,), 0x5b, dtype=torch.uint8, device=dev)
    ops.calib_read_ptq1(W, K, N, w)
    torch.cuda.synchronize()
    assert torch.count_nonzero(w).item() == 0
