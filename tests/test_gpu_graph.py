"""The GEMVs and the prefill GEMM inside HIP graphs (the bench times its decode steps as graph
replays; serving loops capture them the same way): a graph of several launches is replayed
several times with other eager work and synchronisations between the replays, and every
replay's outputs equal the eager launches' bit for bit.  The first call on the capture
stream runs eagerly (scratch buffers are per stream and cannot be allocated under capture)."""
import ctypes

import numpy as np
import pytest
import torch

from kata_amd import ops
from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def _replays_equal_eager(dev, fn, outs, n_replays=4):
    """fn() launches into `outs` (a list of tensors); eager result vs each replay."""
    cs = torch.cuda.Stream(dev)
    with torch.cuda.stream(cs):
        fn()                                         # first call on this stream: eager
    torch.cuda.synchronize()
    ref = [o.clone() for o in outs]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cs):
        fn()
    junk = torch.randn(1 << 20, device=dev)
    for r in range(n_replays):
        for o in outs:
            o.fill_(float("nan") if o.is_floating_point() else -1)   # eager work between the replays
        junk.mul_(1.0001)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs, ref):
            assert torch.equal(o, e), f"replay {r}"


def test_graph_decode_step(dev):
    """The bench's decode step shape: batched GEMVs sharing an input, then single ones,
    several weight sets in one graph."""
    specs = [(5120, (1024, 512)), (6144, (640,)), (5120, (2048, 2048)), (17408, (512,))]
    Ws, xs, ys = [], [], []
    for i, (K, Ns) in enumerate(specs):
        Ws.append([torch.from_numpy(orc.synth_ptq1(N, K, 10 * i + j)[0]).to(dev) for j, N in enumerate(Ns)])
        xs.append(torch.from_numpy(orc.synth_x(1, K, i)).to(dev))
        ys.append([torch.empty((1, N), device=dev) for N in Ns])

    def step():
        for (K, Ns), W, x, y in zip(specs, Ws, xs, ys):
            ops.gemv_ptq1_batch(W, x, K, list(Ns), 1, outs=y)

    _replays_equal_eager(dev, step, [t for y in ys for t in y])


def test_graph_wide_batch_and_t2(dev):
    """The wide verification GEMV (prep + main launch, the stream's image buffer) and the
    T = 2 verify GEMV in one graph."""
    K, Ns = 5120, (3000, 1700)
    Ws = [torch.from_numpy(orc.synth_ptq1(N, K, 40 + j)[0]).to(dev) for j, N in enumerate(Ns)]
    x8 = torch.from_numpy(orc.synth_x(8, K, 41)).to(dev)
    x2 = torch.from_numpy(orc.synth_x(2, K, 42)).to(dev)
    y8 = [torch.empty((8, N), device=dev) for N in Ns]
    y2 = torch.empty((2, Ns[0]), device=dev)

    def calls():
        ops.gemv_ptq1_wide_batch(Ws, x8, K, list(Ns), outs=y8)
        ops.gemv_ptq1(Ws[0], x2, K, Ns[0], 2, out=y2)

    _replays_equal_eager(dev, calls, y8 + [y2])


def test_graph_long_matrix_strided_and_argmax(dev):
    """One long matrix in the tile-strided order, whose items are scaled and stored one item
    later (K = 5120, 66000 rows: >= 64 tiles per workgroup), on the operand form, followed by
    the greedy argmax of its outputs (two launches and the argmax's stream buffer)."""
    K, N = 5120, 66000
    W = torch.from_numpy(orc.synth_ptq1(N, K, 77)[0]).to(dev)
    xq = ops.gemv_prepare_x(torch.from_numpy(orc.synth_x(1, K, 78)).to(dev), K, 1)
    y = torch.empty((1, N), device=dev)
    idx = torch.empty(1, dtype=torch.int32, device=dev)

    def calls():
        ops.gemv_ptq1(W, xq, K, N, 1, out=y)
        ops.argmax(y, out=idx)

    _replays_equal_eager(dev, calls, [y, idx])


def test_graph_prefill_gemm_with_pieces(dev):
    """The fp16 prefill GEMM whose last tile round is split into K pieces (the stream's
    workspace and the piece-sum launch) inside a graph."""
    M, K, N = 300, 2048, 4000
    W = torch.from_numpy(orc.synth_ptq1(N, K, 50)[0]).to(dev)
    A = torch.from_numpy(orc.synth_x(M, K, 51)).to(dev)
    C = torch.empty((M, N), dtype=torch.float16, device=dev)
    _replays_equal_eager(dev, lambda: ops.gemm_ptq1_f16(A, W, K, N, out=C), [C])


def test_graph_replay_after_scratch_grows(dev):
    """A graph captured with a small wide-GEMV image (K = 5120), then an eager call on the same
    stream that needs a larger image (K = 17408): the replays still read the buffer the graph
    recorded (the outgrown buffer is retired, not freed) and equal the eager results bit for
    bit; kata_release_stream then frees the stream's buffers and a later call reallocates."""
    from kata_amd.capi import check, lib
    Ks, Ns = (5120, 17408), (2000, 1100)
    Ws = [torch.from_numpy(orc.synth_ptq1(N, K, 60 + i)[0]).to(dev) for i, (K, N) in enumerate(zip(Ks, Ns))]
    xs = [torch.from_numpy(orc.synth_x(8, K, 62 + i)).to(dev) for i, K in enumerate(Ks)]
    ys = [torch.empty((8, N), device=dev) for N in Ns]
    cs = torch.cuda.Stream(dev)
    with torch.cuda.stream(cs):
        ops.gemv_ptq1_wide(Ws[0], xs[0], Ks[0], Ns[0], out=ys[0])      # eager: image for K = 5120
    torch.cuda.synchronize()
    ref_small = ys[0].clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cs):
        ops.gemv_ptq1_wide(Ws[0], xs[0], Ks[0], Ns[0], out=ys[0])
    for r in range(3):
        with torch.cuda.stream(cs):
            ops.gemv_ptq1_wide(Ws[1], xs[1], Ks[1], Ns[1], out=ys[1])  # eager: grows the image
        torch.cuda.synchronize()
        big = ys[1].clone()
        ys[0].fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(ys[0], ref_small), f"replay {r} after the buffer grew"
        if r:
            assert torch.equal(ys[1], big)
    del g
    torch.cuda.synchronize()
    check(lib().kata_release_stream(ctypes.c_void_p(cs.cuda_stream)))
    with torch.cuda.stream(cs):
        ops.gemv_ptq1_wide(Ws[0], xs[0], Ks[0], Ns[0], out=ys[0])      # reallocates
    torch.cuda.synchronize()
    assert torch.equal(ys[0], ref_small)


def test_graph_dispatcher_operand_paths_capture_first(dev):
    """The dispatcher's decode and verify FFN sublayers keep their activations in the GEMVs'
    operand form and allocate nothing: they are captured on a fresh stream with no eager call
    before (an allocation under capture would fail the capture), and every replay equals an
    eager run on another stream bit for bit."""
    from kata_amd.engine import Dispatch
    from kata_amd.capi import lib
    H, F = 2048, 3072
    Wg, _, _ = orc.synth_ptq1(F, H, 71)
    Wu, _, _ = orc.synth_ptq1(F, H, 72)
    Wd, _, _ = orc.synth_ptq1(H, F, 73)
    buf = np.concatenate([Wg.ravel(), Wu.ravel(), Wd.ravel()])
    offs = (0, Wg.size, Wg.size + Wu.size)
    d = Dispatch(torch.from_numpy(buf).to(dev))
    rng = np.random.default_rng(5)
    t = lambda a: torch.from_numpy(a.astype(np.float32)).to(dev)
    gs_in, gs_down = t(rng.choice([-1.0, 1.0], H)), t(rng.choice([-1.0, 1.0], F))
    cases = []
    for T in (1, 3, 8):
        x, y = t(rng.standard_normal((T, H))), t(0.3 * rng.standard_normal((T, H)))
        out, xnew = torch.empty((T, H), device=dev), torch.empty((T, H), device=dev)
        if T == 1:
            work = torch.empty(H + 3 * F, dtype=torch.float32, device=dev)
            fn = (lambda x=x, y=y, out=out, xnew=xnew, work=work:
                  d.ffn_decode(*offs, x[0], y[0], gs_in, gs_down, H, F, out=out[0], xnew=xnew[0], work=work))
        else:
            work = torch.empty(int(lib().kata_ffn_verify_work_bytes(H, F, T)), dtype=torch.uint8, device=dev)
            fn = (lambda x=x, y=y, out=out, xnew=xnew, work=work:
                  d.ffn_verify(*offs, x, y, gs_in, gs_down, H, F, out=out, xnew=xnew, work=work))
        cases.append((fn, out))
    cs = torch.cuda.Stream(dev)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cs):
        for fn, _ in cases:
            fn()
    es = torch.cuda.Stream(dev)
    with torch.cuda.stream(es):
        for fn, _ in cases:
            fn()
    torch.cuda.synchronize()
    ref = [o.clone() for _, o in cases]
    for r in range(3):
        for _, o in cases:
            o.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for (_, o), e in zip(cases, ref):
            assert torch.equal(o, e), f"replay {r}"
