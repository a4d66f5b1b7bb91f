#!/usr/bin/env python3
"""Benchmark of the MI355X ternary-matmul hot path (one GPU).

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu] [--no-gemm]

Workload (the batch-1 decode sweep): one step is the T=1 decode
GEMV of every ternary matrix of one layer of each kind at the 27B shapes —
GDN qkv 5120->10240, z 5120->6144, ssm_out 6144->5120; GQA q 5120->12288, k/v 5120->1024,
o 6144->5120; FFN gate/up 5120->17408, down 17408->5120.  The matrices that multiply the
same input run as one launch (kata_gemv_ptq1_batch: qkv+z, q+k+v, gate+up; ssm_out, o and
down alone), 6 launches per step.  The GEMVs take each input in the operand form (KATA_XQ:
the activation quantised to the kernel's 16-bit block fixed point and laid out as its
matrix-core operand), which in the model the input transform writes in place of fp32 rows
(kata_add_rms_fwht / kata_rms_fwht with out_dtype KATA_XQ, the dispatcher's decode form);
it is prepared once before the timed region, as the reference's GEMV is timed on an
activation its rms_fwht kernel already wrote.  `raw_x_step` times the same step on fp16 rows,
each GEMV workgroup quantising them itself, and input_transform times the transform with
either output.
Weights are seeded
synthetic PTQ1_0 (trits iid on {-1,0,1}, fp16 scales |N(0,0.02)|), activations fp16
N(0,1).  Steps rotate over enough distinct weight copies (>= 512 MB) that no matrix is
served from the 256 MB Infinity Cache.  `value` = packed weight bytes of all GEMVs of the
timed steps / wall time of those steps (events on the launch stream), in GB/s; a step's 6
launches are captured as HIP graphs, one per timed batch of steps, and replayed (--launch host
issues every GEMV from Python instead; both figures are in the JSON line).

Also reported (same JSON line):
  roofline     dominant kernel k_gemv_ptq1<1>: algorithmic bytes per launch (the packed
               weight bytes, averaged over the sweep's matrices) / its average launch
               duration, vs 8 TB/s HBM;
  per_matrix   GB/s of each matrix kind alone (200 repeats over rotating copies, replayed
               from one HIP graph so that the host's launch cost is not what is timed);
  verify_t2    config 3: the T=2 verify GEMV on the FFN and attention shapes;
  verify_wide  the wide verification GEMV (T = 4, 8 token rows) on the same shapes;
  q8_0_t1      config 3: the Q8_0 MTP-head GEMV, 17408x5120 and 5120x17408;
  prefill_gemm pp512 exact fp16 GEMM TFLOPS (M=512, 5120->17408 and 17408->5120),
               vs 2.5 PFLOP/s dense fp16, the int8 variant, and the Q8_0 MTP K/V catch-up
               GEMM (eh_proj 10240->5120, wk 5120->1024, M=512);
  cpu_baseline the reference's host path for BASELINE config 1 (the full 17408x5120 matrix:
               stage-loop dequantize_row_ptq1_0 + fp32 dot,
               oracle/kata_oracle.c:orc_cpu_gemv_ptq1_stage) on all host cores this process
               may use (nproc and the thread count stated), and on one thread.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0
WARM_MS = 25.0          # back-to-back replays before each timed replay (see graph_time)
FP16_PEAK_TFLOPS = 2500.0
INT8_PEAK_TOPS = 5000.0

# (name, K, N, input) of one layer of each kind; matrices of one input share its activation
SWEEP = [
    ("gdn_qkv", 5120, 10240, "gdn_in"), ("gdn_z", 5120, 6144, "gdn_in"), ("gdn_ssm_out", 6144, 5120, "gdn_out"),
    ("attn_q", 5120, 12288, "attn_in"), ("attn_k", 5120, 1024, "attn_in"), ("attn_v", 5120, 1024, "attn_in"),
    ("attn_o", 6144, 5120, "attn_out"),
    ("ffn_gate", 5120, 17408, "ffn_in"), ("ffn_up", 5120, 17408, "ffn_in"), ("ffn_down", 17408, 5120, "ffn_mid"),
]
SEED = 20260501


def packed_bytes(K, N):
    return N * (K // 128) * 28


def make_weights(torch, dev, K, N, seed, ops):
    """One packed matrix built on the host with the library's packer, then on device."""
    rng = np.random.default_rng(seed)
    trits = rng.integers(-1, 2, size=(N, K), dtype=np.int8)
    scales = np.abs(rng.normal(0.0, 0.02, size=(N, K // 128))).astype(np.float16)
    return torch.from_numpy(ops.pack_ptq1(trits, scales)).to(dev)


def device_weights(torch, dev, K, N, gen):
    """A packed PTQ1_0 matrix drawn on the device with the same distribution: iid uniform
    trits are iid uniform qs bytes in [0, 243) and qh bytes in [0, 81); d = fp16 |N(0, 0.02)|."""
    nb = K // 128
    blk = torch.empty((N, nb, 28), dtype=torch.uint8, device=dev)
    blk[:, :, :24] = torch.randint(0, 243, (N, nb, 24), generator=gen, device=dev, dtype=torch.uint8)
    blk[:, :, 24:26] = torch.randint(0, 81, (N, nb, 2), generator=gen, device=dev, dtype=torch.uint8)
    d = (torch.randn((N, nb), generator=gen, device=dev) * 0.02).abs().half()
    blk[:, :, 26:28] = d.view(torch.uint8).view(N, nb, 2)
    return blk.view(N, nb * 28)


# 64-layer trunk of the 27B model (48 gated-DeltaNet + 16 GQA layers, each with an FFN) and
# the lm_head, as the decode step launches them (inputs shared by qkv+z, q+k+v, gate+up)
GDN_LAUNCHES = [(5120, (10240, 6144)), (6144, (5120,)), (5120, (17408, 17408)), (17408, (5120,))]
GQA_LAUNCHES = [(5120, (12288, 1024, 1024)), (6144, (5120,)), (5120, (17408, 17408)), (17408, (5120,))]
LM_HEAD = (5120, (248320,))


def run_config5(torch, ops, dev, stream):
    """one bs=1 decode pass over all 64 layers + lm_head (5.6 GB of
    ternary weights, far above the Infinity Cache) and the 7300-token prefill GEMMs (as one
    GEMM and as 1024-row chunks), fp16 exact and int8 paths."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(SEED + 900)
    layers = [GDN_LAUNCHES] * 48 + [GQA_LAUNCHES] * 16
    launches = [(K, [device_weights(torch, dev, K, N, gen) for N in Ns], Ns) for L in layers for K, Ns in L]
    launches.append((LM_HEAD[0], [device_weights(torch, dev, LM_HEAD[0], LM_HEAD[1][0], gen)], LM_HEAD[1]))
    total = sum(w.numel() for _, ws, _ in launches for w in ws)
    xs = {K: ops.gemv_prepare_x(torch.randn((1, K), generator=gen, device=dev).half(), K, 1) for K in (5120, 6144, 17408)}
    ys = {N: torch.empty((1, N), dtype=torch.float32, device=dev) for N in (1024, 5120, 6144, 10240, 12288, 17408, 248320)}

    def sweep():
        for K, ws, Ns in launches:
            if len(ws) == 1:
                ops.gemv_ptq1(ws[0], xs[K], K, Ns[0], 1, out=ys[Ns[0]])
            else:
                ops.gemv_ptq1_batch(ws, xs[K], K, list(Ns), 1, outs=[ys[N] for N in Ns])
    sweep()
    torch.cuda.synchronize()
    # the pass captured once as a HIP graph (as a serving loop runs its decode step) and, for
    # comparison, launched from the host
    cs = torch.cuda.Stream(dev)
    with torch.cuda.stream(cs):
        sweep()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cs):
        sweep()
    g.replay()
    torch.cuda.synchronize()

    def median_ms(run):
        # >= WARM_MS of back-to-back passes, then five timed ones, events between them and no
        # host synchronisation (the clock drops while the GPU idles)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        run()
        b.record(stream)
        torch.cuda.synchronize()
        for _ in range(math.ceil(WARM_MS / max(a.elapsed_time(b), 1e-3))):
            run()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(6)]
        ev[0].record(stream)
        for i in range(5):
            run()
            ev[i + 1].record(stream)
        torch.cuda.synchronize()
        times = [ev[i].elapsed_time(ev[i + 1]) for i in range(5)]
        return sorted(times)[len(times) // 2]

    ms = median_ms(g.replay)
    ms_host = median_ms(sweep)
    del g
    out = {"decode_64_layers": {"bytes": total, "launches": len(launches), "ms_median_of_5": round(ms, 3),
                                "GBps": round(total / (ms * 1e-3) / 1e9, 1), "launch": "graph",
                                "host_launch_ms": round(ms_host, 3),
                                "host_launch_GBps": round(total / (ms_host * 1e-3) / 1e9, 1)}}
    del launches
    # 7300-token prefill, gate and down shapes
    M = 7300
    pre = {}
    for name, K, N in (("ffn_gate", 5120, 17408), ("ffn_down", 17408, 5120)):
        W = device_weights(torch, dev, K, N, gen)
        A = torch.randn((M, K), generator=gen, device=dev).half()
        C = torch.empty((M, N), dtype=torch.float16, device=dev)
        Q = torch.empty((M, K), dtype=torch.int8, device=dev)
        SX = torch.empty((K // 128, M), dtype=torch.float32, device=dev)

        def timed(fn, nrep=5):
            sustain(torch, fn, stream)
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(stream)
            for _ in range(nrep):
                fn()
            b.record(stream)
            torch.cuda.synchronize()
            return a.elapsed_time(b) * 1e3 / nrep

        def chunks_f16():
            for m0 in range(0, M, 1024):
                ops.gemm_ptq1_f16(A[m0:m0 + 1024], W, K, N, out=C[m0:m0 + 1024])

        us = timed(lambda: ops.gemm_ptq1_f16(A, W, K, N, out=C))
        us_c = timed(chunks_f16)
        ops.quant_rows(A, out=(Q, SX))
        us_i8 = timed(lambda: ops.gemm_ptq1_i8(Q, SX, W, K, N, out=C))
        fl = 2.0 * M * N * K
        pre[name] = {"M": M, "K": K, "N": N, "f16_us": round(us, 1), "f16_TFLOPS": round(fl / (us * 1e-6) / 1e12, 1),
                     "f16_1024_chunks_us": round(us_c, 1),
                     "i8_us": round(us_i8, 1), "i8_TOPS": round(fl / (us_i8 * 1e-6) / 1e12, 1)}
        del W, A, C, Q, SX
    out["prefill_m7300"] = pre
    torch.cuda.empty_cache()
    return out


def cpu_baseline(threads: int, reps: int = 3):
    """BASELINE config 1 on the host: the full 17408x5120 gate matrix, each row expanded by the
    reference's stage-loop dequantize_row_ptq1_0 then fp32 dots (orc_cpu_gemv_ptq1_stage),
    OpenMP over rows; best of `reps` runs, GB/s of packed bytes."""
    from oracle import oracle as orc
    K, N = 5120, 17408
    W, _, _ = orc.synth_ptq1(N, K, SEED + 1000)
    x = orc.synth_x(1, K, SEED + 2000).astype(np.float32)
    best = float("inf")
    for _ in range(reps):
        t0 = time.perf_counter()
        orc.cpu_gemv_stage(W, x, K, N, 1, 0, N, threads)
        best = min(best, time.perf_counter() - t0)
    return packed_bytes(K, N) / best / 1e9, packed_bytes(K, N)


def cpu_gemm_baseline(threads: int, rows: int = 512):
    """The pp512 gate GEMM on the host (decode each weight row to fp32 once, fp32 dots against
    the 512 activation rows, OpenMP over weight rows) on its first `rows` weight rows."""
    from oracle import oracle as orc
    M, K, N = 512, 5120, 17408
    W, _, _ = orc.synth_ptq1(rows, K, SEED + 3000)
    A = orc.synth_x(M, K, SEED + 3001)
    out = {"unit": "GFLOP/s", "sample": f"M={M}, K={K}, first {rows} of the N={N} gate rows"}
    for key, th in (("value", threads), ("single_thread", 1)):
        t0 = time.perf_counter()
        orc.cpu_gemm_f32(A, W, M, K, rows, 0, rows, th)
        out[key] = round(2.0 * M * K * rows / (time.perf_counter() - t0) / 1e9, 2)
    out["cores"] = threads
    return out


def sustain(torch, fn, stream, ms=200.0):
    """Calls fn until the GPU has run it for `ms` milliseconds (event-timed).  Under sustained
    matrix-core load the clock settles over tens of milliseconds: a GEMM timed after a few
    warm-up calls reads about 15 % slower than the steady state a prefill runs at (a GEMV
    settles within a few milliseconds of back-to-back work: graph_time's warm-up)."""
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    total, n = 0.0, 1
    while total < ms:
        a.record(stream)
        for _ in range(n):
            fn()
        b.record(stream)
        torch.cuda.synchronize()
        total += a.elapsed_time(b)
        n = min(2 * n, 64)


def run_gemm(torch, ops, dev, stream, copies, ncopies):
    """pp512 exact fp16 prefill GEMM (config 4): us and TFLOPS per shape, 30 calls over
    rotating weight copies between two events, after 200 ms of sustained calls."""
    gemm = {}
    M = 512
    A = {K: torch.from_numpy(np.random.default_rng(K).standard_normal((M, K)).astype(np.float16)).to(dev)
         for K in (5120, 17408)}
    for name, K, N, j in (("ffn_gate", 5120, 17408, 7), ("ffn_down", 17408, 5120, 9)):
        C = torch.empty((M, N), dtype=torch.float16, device=dev)
        sustain(torch, lambda: ops.gemm_ptq1_f16(A[K], copies[0][j], K, N, out=C), stream)
        nrep = 30
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for r in range(nrep):
            ops.gemm_ptq1_f16(A[K], copies[r % ncopies][j], K, N, out=C)
        b.record(stream)
        torch.cuda.synchronize()
        us = a.elapsed_time(b) * 1e3 / nrep
        tflops = 2.0 * M * N * K / (us * 1e-6) / 1e12
        gemm[name] = {"M": M, "K": K, "N": N, "us": round(us, 1), "TFLOPS": round(tflops, 1),
                      "frac": round(tflops / FP16_PEAK_TFLOPS, 4)}
        # the int8 FFN variant (config 5): activation quantisation + int8 GEMM
        Q, SX = ops.quant_rows(A[K])
        sustain(torch, lambda: ops.gemm_ptq1_i8(Q, SX, copies[0][j], K, N, out=C), stream)
        a.record(stream)
        for r in range(nrep):
            ops.quant_rows(A[K], out=(Q, SX))
        b.record(stream)
        torch.cuda.synchronize()
        us_q = a.elapsed_time(b) * 1e3 / nrep
        a.record(stream)
        for r in range(nrep):
            ops.gemm_ptq1_i8(Q, SX, copies[r % ncopies][j], K, N, out=C)
        b.record(stream)
        torch.cuda.synchronize()
        us_i = a.elapsed_time(b) * 1e3 / nrep
        tops = 2.0 * M * N * K / (us_i * 1e-6) / 1e12
        gemm[name + "_i8"] = {"M": M, "K": K, "N": N, "quant_us": round(us_q, 1), "us": round(us_i, 1),
                              "TOPS": round(tops, 1), "frac": round(tops / INT8_PEAK_TOPS, 4)}
    # the MTP head's K/V catch-up over Q8_0 weights (eh_proj 10240 -> 5120, wk 5120 -> 1024),
    # over two weight copies (eh_proj: 2 x 55.7 MB, past the L2s)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for name, K, N in (("mtp_eh_proj_q8", 10240, 5120), ("mtp_wk_q8", 5120, 1024)):
        rng = np.random.default_rng(K + N)
        blk = rng.integers(-127, 128, size=(N, K // 32, 34), dtype=np.int64).astype(np.int8).view(np.uint8)
        blk[:, :, 0:2] = np.abs(rng.normal(0.0, 0.02, size=(N, K // 32))).astype(np.float16).view(np.uint8).reshape(
            N, K // 32, 2)
        Wq = [torch.from_numpy(np.ascontiguousarray(blk).reshape(N, -1)).to(dev) for _ in range(2)]
        Aq = torch.from_numpy(np.random.default_rng(K + 1).standard_normal((M, K)).astype(np.float16)).to(dev)
        C = torch.empty((M, N), dtype=torch.float16, device=dev)
        sustain(torch, lambda: ops.gemm_q8_f16(Aq, Wq[0], K, N, out=C), stream)
        nrep = 30
        a.record(stream)
        for r in range(nrep):
            ops.gemm_q8_f16(Aq, Wq[r % 2], K, N, out=C)
        b.record(stream)
        torch.cuda.synchronize()
        us = a.elapsed_time(b) * 1e3 / nrep
        tflops = 2.0 * M * N * K / (us * 1e-6) / 1e12
        gemm[name] = {"M": M, "K": K, "N": N, "us": round(us, 1), "TFLOPS": round(tflops, 1),
                      "frac": round(tflops / FP16_PEAK_TFLOPS, 4)}
        del Wq
    return gemm


def graph_time(torch, fn, nrep, stream, cap_stream, warm_ms=WARM_MS):
    """us per call of fn(r), r = 0..nrep-1, captured once into a graph and replayed: the
    host's per-launch cost (a Python call each) stays out of the timed region.  The warm-up
    calls run on the capture stream: scratch buffers are per stream and are allocated by a
    stream's first call, which cannot happen inside the capture.  The timed replay follows
    at least warm_ms of back-to-back replays with no host synchronisation in between: after
    the GPU idles (graph capture, allocation) its clock drops, and the first milliseconds of
    work read up to 25 % slower (lm_head 84.8 against 67 us; the plain read ~4 %)."""
    with torch.cuda.stream(cap_stream):
        for r in range(3):
            fn(r)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cap_stream):
        for r in range(nrep):
            fn(r)
    g.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    g.replay()
    b.record(stream)
    torch.cuda.synchronize()
    for _ in range(max(1, math.ceil(warm_ms / max(a.elapsed_time(b), 1e-3)))):
        g.replay()
    a.record(stream)
    g.replay()
    b.record(stream)
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e3 / nrep


def run_ffn(torch, ops, dev, stream, time_reps):
    """The FFN sublayer at the 27B shapes (H=5120, F=17408) through the dispatcher: decode
    (4 launches) over 8 rotating weight sets (470 MB, past the MALL), T=8 verification,
    pp512 prefill."""
    from kata_amd.engine import Dispatch, ffn_prefill_work_bytes
    H, F = 5120, 17408
    gen = torch.Generator(device=dev)
    gen.manual_seed(SEED + 800)
    nset = 8
    mats = []
    for _ in range(nset):
        mats += [device_weights(torch, dev, H, F, gen), device_weights(torch, dev, H, F, gen),
                 device_weights(torch, dev, F, H, gen)]
    wbuf = torch.cat([m.reshape(-1) for m in mats])
    del mats
    msz = [packed_bytes(H, F), packed_bytes(H, F), packed_bytes(F, H)]
    set_b = sum(msz)
    disp = Dispatch(wbuf)
    offs = lambda r: (set_b * (r % nset), set_b * (r % nset) + msz[0], set_b * (r % nset) + msz[0] + msz[1])
    fx = torch.randn(H, generator=gen, device=dev)
    fy = torch.randn(H, generator=gen, device=dev)
    fxn = torch.empty(H, device=dev)
    gsi = torch.randn(H, generator=gen, device=dev).sign()
    gsd = torch.randn(F, generator=gen, device=dev).sign()
    fout = torch.empty(H, device=dev)
    fwork = torch.empty(H + 3 * F, device=dev)
    us_d = time_reps(lambda r: disp.ffn_decode(*offs(r), fx, fy, gsi, gsd, H, F, out=fout, xnew=fxn,
                                               work=fwork), 40)
    ffn = {"H": H, "F": F, "decode_us": round(us_d, 2),
           "decode_GBps": round(set_b / (us_d * 1e-6) / 1e9, 1)}
    # T = 8 verification tokens: transform, batched gate + up, SwiGLU transform, down
    Tv = 8
    vx = torch.randn((Tv, H), generator=gen, device=dev)
    vy = torch.randn((Tv, H), generator=gen, device=dev)
    vxn = torch.empty((Tv, H), device=dev)
    vout = torch.empty((Tv, H), device=dev)
    vwork = torch.empty(int(ops.lib().kata_ffn_verify_work_bytes(H, F, Tv)), dtype=torch.uint8, device=dev)
    us_v = time_reps(lambda r: disp.ffn_verify(*offs(r), vx, vy, gsi, gsd, H, F, out=vout, xnew=vxn,
                                               work=vwork), 40)
    ffn["verify_t8_us"] = round(us_v, 2)
    ffn["verify_t8_GBps"] = round(set_b / (us_v * 1e-6) / 1e9, 1)
    M = 512
    px = torch.randn((M, H), generator=gen, device=dev)
    py = torch.randn((M, H), generator=gen, device=dev)
    pxn = torch.empty((M, H), device=dev)
    pout = torch.empty((M, H), device=dev)
    pwork = torch.empty(ffn_prefill_work_bytes(H, F, M), dtype=torch.uint8, device=dev)
    for spec in ("none", "ffn"):
        disp.set_i8(spec)
        sustain(torch, lambda: disp.ffn_prefill(*offs(0), px, py, gsi, gsd, H, F, out=pout, xnew=pxn,
                                                work=pwork), stream)
        us_p = time_reps(lambda r: disp.ffn_prefill(*offs(r), px, py, gsi, gsd, H, F, out=pout, xnew=pxn,
                                                    work=pwork), 10)
        ffn[f"prefill_m512_i8_{spec}_us"] = round(us_p, 1)
        ffn[f"prefill_m512_i8_{spec}_TFLOPS"] = round(2 * M * 3 * H * F / (us_p * 1e-6) / 1e12, 1)
    disp.close()
    del wbuf, disp
    return ffn


def run_q8(torch, ops, dev, time_reps, reps):
    """Config 3: the Q8_0 MTP-head GEMV at 17408x5120 and 5120x17408, one and two activation
    rows, over rotating weight copies (> 512 MB)."""
    q8 = {}
    for name, K, N in (("gate", 5120, 17408), ("down", 17408, 5120)):
        nb = N * (K // 32) * 34
        nq8 = max(2, -(-512 * 1024 * 1024 // nb))
        rng = np.random.default_rng(SEED + 400 + K)
        blk = rng.integers(-127, 128, size=(N, K // 32, 34), dtype=np.int64).astype(np.int8).view(np.uint8)
        d = np.abs(rng.normal(0.0, 0.02, size=(N, K // 32))).astype(np.float16).view(np.uint8).reshape(N, K // 32, 2)
        blk[:, :, 0:2] = d
        Wq = torch.from_numpy(np.ascontiguousarray(blk).reshape(N, -1)).to(dev)
        Wqs = [Wq] + [Wq.clone() for _ in range(nq8 - 1)]
        xq = torch.from_numpy(np.random.default_rng(SEED + 500 + K).standard_normal((1, K))
                              .astype(np.float16)).to(dev)
        yq = torch.empty((1, N), dtype=torch.float32, device=dev)
        us = time_reps(lambda r: ops.gemv_q8(Wqs[r % nq8], xq, K, N, 1, out=yq), max(20, reps // 4))
        q8[name] = {"K": K, "N": N, "us": round(us, 3), "GBps": round(nb / (us * 1e-6) / 1e9, 1)}
        # the MTP head's two-row form (mtpRows, R = 2): both rows per weight read
        xq2 = torch.from_numpy(np.random.default_rng(SEED + 600 + K).standard_normal((2, K))
                               .astype(np.float16)).to(dev)
        yq2 = torch.empty((2, N), dtype=torch.float32, device=dev)
        us2 = time_reps(lambda r: ops.gemv_q8(Wqs[r % nq8], xq2, K, N, 2, out=yq2), max(20, reps // 4))
        q8[name].update({"t2_us": round(us2, 3), "t2_GBps": round(nb / (us2 * 1e-6) / 1e9, 1)})
        del Wqs, Wq
    # the MTP block's shared-input launches (src/engine.cpp:361,369): wq + wk + wv and gate + up
    # as one batched launch against their separate launches, one activation row
    def q8_mat(N, K, seed):
        rng = np.random.default_rng(seed)
        blk = rng.integers(-127, 128, size=(N, K // 32, 34), dtype=np.int64).astype(np.int8).view(np.uint8)
        blk[:, :, 0:2] = np.abs(rng.normal(0.0, 0.02, size=(N, K // 32))).astype(np.float16).view(np.uint8).reshape(N, K // 32, 2)
        return torch.from_numpy(np.ascontiguousarray(blk).reshape(N, -1)).to(dev)
    xq = torch.from_numpy(np.random.default_rng(SEED + 700).standard_normal((1, 5120)).astype(np.float16)).to(dev)
    for name, Ns in (("wq_wk_wv", (12288, 1024, 1024)), ("gate_up", (17408, 17408))):
        nb = sum(N * (5120 // 32) * 34 for N in Ns)
        ncp = max(2, -(-512 * 1024 * 1024 // nb))
        sets = [[q8_mat(N, 5120, SEED + 800 + 7 * i) for i, N in enumerate(Ns)]]
        sets += [[w.clone() for w in sets[0]] for _ in range(ncp - 1)]
        ys = [torch.empty((1, N), dtype=torch.float32, device=dev) for N in Ns]
        us_b = time_reps(lambda r: ops.gemv_q8_batch(sets[r % ncp], xq, 5120, list(Ns), 1, outs=ys), max(20, reps // 4))

        def separate(r):
            for w, y, N in zip(sets[r % ncp], ys, Ns):
                ops.gemv_q8(w, xq, 5120, N, 1, out=y)
        us_s = time_reps(separate, max(20, reps // 4))
        q8[name] = {"K": 5120, "N": list(Ns), "batched_us": round(us_b, 3), "batched_GBps": round(nb / (us_b * 1e-6) / 1e9, 1),
                    "separate_us": round(us_s, 3), "separate_GBps": round(nb / (us_s * 1e-6) / 1e9, 1)}
        del sets
    return q8


def run_verify_wide(torch, ops, dev, copies, ncopies, time_reps, reps):
    """The wide verification GEMV (Engine::dWide) at T = 4 and 8 token rows on the FFN and
    attention shapes (one weight read for all rows), and verifyWide's gate + up batched: on
    the operand form of the rows (what the dispatcher's transforms write; t{T}_us) and on fp16
    rows, quantised by a prep launch first (t{T}_raw_us)."""
    # wide verification GEMV (Engine::dWide): T = 4 and 8 token rows, one weight read
    verify_wide = {}
    for j, (name, K, N, grp) in enumerate(SWEEP):
        if name not in ("gdn_qkv", "attn_q", "attn_o", "ffn_gate", "ffn_down"):
            continue
        ent = {"K": K, "N": N}
        for T in (4, 8):
            xw = torch.from_numpy(np.random.default_rng(SEED + 350 + j).standard_normal((T, K))
                                  .astype(np.float16)).to(dev)
            yw = torch.empty((T, N), dtype=torch.float32, device=dev)
            xq = ops.gemv_prepare_x(xw, K, T)
            us = time_reps(lambda r: ops.gemv_ptq1_wide(copies[r % ncopies][j], xq, K, N, out=yw, T=T), reps)
            us_raw = time_reps(lambda r: ops.gemv_ptq1_wide(copies[r % ncopies][j], xw, K, N, out=yw), reps)
            ent[f"t{T}_us"] = round(us, 3)
            ent[f"t{T}_GBps"] = round(packed_bytes(K, N) / (us * 1e-6) / 1e9, 1)
            ent[f"t{T}_raw_us"] = round(us_raw, 3)
        verify_wide[name] = ent
    # verifyWide's gate + up in one batched launch (one quantisation of the token rows)
    jg, ju = [i for i, e in enumerate(SWEEP) if e[0] in ("ffn_gate", "ffn_up")]
    K, N = SWEEP[jg][1], SWEEP[jg][2]
    ent = {"K": K, "N": 2 * N}
    for T in (4, 8):
        xw = torch.from_numpy(np.random.default_rng(SEED + 360).standard_normal((T, K)).astype(np.float16)).to(dev)
        ygu = [torch.empty((T, N), dtype=torch.float32, device=dev) for _ in range(2)]
        xq = ops.gemv_prepare_x(xw, K, T)
        us = time_reps(lambda r: ops.gemv_ptq1_wide_batch([copies[r % ncopies][jg], copies[r % ncopies][ju]], xq, K,
                                                          [N, N], outs=ygu, T=T), reps)
        us_raw = time_reps(lambda r: ops.gemv_ptq1_wide_batch([copies[r % ncopies][jg], copies[r % ncopies][ju]], xw,
                                                              K, [N, N], outs=ygu), reps)
        ent[f"t{T}_us"] = round(us, 3)
        ent[f"t{T}_raw_us"] = round(us_raw, 3)
        ent[f"t{T}_GBps"] = round(2 * packed_bytes(K, N) / (us * 1e-6) / 1e9, 1)
    verify_wide["ffn_gate_up_batched"] = ent
    return verify_wide


def run_lm_head(torch, ops, dev, lx, time_reps):
    """The lm_head GEMV (5120 -> 248320, 278 MB; two weight copies, 556 MB, past the MALL) on
    the operand form lx, the greedy argmax of its logits, and the GEMV's weight-load stream
    alone (kata_calib_read_ptq1) on the same weights."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(SEED + 700)
    lm = [device_weights(torch, dev, 5120, 248320, gen) for _ in range(2)]
    ly = torch.empty((1, 248320), dtype=torch.float32, device=dev)
    lidx = torch.empty(1, dtype=torch.int32, device=dev)
    cw = torch.zeros(4, dtype=torch.int32, device=dev)
    us_lm = time_reps(lambda r: ops.gemv_ptq1(lm[r % 2], lx, 5120, 248320, 1, out=ly), 40)
    us_am = time_reps(lambda r: ops.argmax(ly, out=lidx), 40)
    us_lws = time_reps(lambda r: ops.calib_read_ptq1(lm[r % 2], 5120, 248320, cw), 40)
    nbytes = lm[0].numel()
    del lm
    return {"K": 5120, "N": 248320, "gemv_us": round(us_lm, 2), "GBps": round(nbytes / (us_lm * 1e-6) / 1e9, 1),
            "argmax_us": round(us_am, 2), "weight_stream_us": round(us_lws, 2),
            "weight_stream_GBps": round(nbytes / (us_lws * 1e-6) / 1e9, 1),
            "vs_weight_stream": round(us_lm / us_lws, 3)}


def run_calib_sweep(torch, ops, dev, stream, cap_stream):
    """The plain read at the sweep's sizes over every geometry of kata_calib_read_cfg:
    threads 256/512/1024 x workgroups per CU 1/2/4/8 (<= 2048 threads per CU) x loads in
    flight 2/4/8/16 x non-temporal hint off/on, graph-replayed over rotating buffers (>= 512
    MB per size); per size every configuration's us and the best."""
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    cword = torch.zeros(4, dtype=torch.int32, device=dev)
    out = {}
    for label, nbytes in (("19.5MB", packed_bytes(5120, 17408)), ("39MB", 2 * packed_bytes(5120, 17408)),
                          ("278MB", packed_bytes(5120, 248320))):
        nb = max(2, -(-512 * 1024 * 1024 // nbytes))
        bufs = [torch.empty(nbytes, dtype=torch.uint8, device=dev) for _ in range(nb)]
        for b_ in bufs:
            b_.fill_(1)
        reps = 100 if nbytes < 1e8 else 20
        res = {}
        for threads in (256, 512, 1024):
            for wpc in (1, 2, 4, 8):
                if threads * wpc > 2048:
                    continue
                for inflight in (2, 4, 8, 16):
                    for nt in (False, True):
                        us = graph_time(torch, lambda r: ops.calib_read_cfg(bufs[r % nb], cword, threads, cus * wpc,
                                                                            inflight, nt), reps, stream, cap_stream)
                        res[f"{threads}x{wpc} d{inflight}{' nt' if nt else ''}"] = round(us, 3)
        best = min(res, key=res.get)
        out[label] = {"bytes": nbytes, "best": best, "best_us": res[best],
                      "best_GBps": round(nbytes / (res[best] * 1e-6) / 1e9, 1), "all_us": res}
        del bufs
    return out


def run_calibration(torch, ops, dev, stream, cap_stream, reps):
    """The launch floor of an empty kernel at the decode GEMV's geometry and a plain streaming
    read at the sweep's sizes (same protocol as per_matrix), over rotating buffers (>= 512 MB
    per size) so that reads come from HBM: `read` at the GEMV's geometry (one 1024-thread
    workgroup per CU, ordinary loads), `peak` at the fastest plain-read geometry found
    (two 256-thread workgroups per CU, non-temporal loads) -- the read ceiling."""
    calib = {}
    cword = torch.zeros(4, dtype=torch.int32, device=dev)
    calib["empty_us"] = round(graph_time(torch, lambda r: ops.calib_empty(cword), reps, stream, cap_stream), 3)
    for label, nbytes in (("19.5MB", packed_bytes(5120, 17408)), ("39MB", 2 * packed_bytes(5120, 17408)),
                          ("278MB", packed_bytes(5120, 248320))):
        nb = max(2, -(-512 * 1024 * 1024 // nbytes))
        bufs = [torch.empty(nbytes, dtype=torch.uint8, device=dev) for _ in range(nb)]
        for b_ in bufs:
            b_.fill_(1)
        n = reps if nbytes < 1e8 else 40
        us = graph_time(torch, lambda r: ops.calib_read(bufs[r % nb], cword), n, stream, cap_stream)
        up = graph_time(torch, lambda r: ops.calib_read_peak(bufs[r % nb], cword), n, stream, cap_stream)
        calib[label] = {"bytes": nbytes, "us": round(us, 3), "GBps": round(nbytes / (us * 1e-6) / 1e9, 1),
                        "peak_us": round(up, 3), "peak_GBps": round(nbytes / (up * 1e-6) / 1e9, 1)}
        del bufs
    return calib


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-gemm", action="store_true")
    ap.add_argument("--launch", choices=("graph", "host"), default="graph",
                    help="graph: each timed batch of steps is captured once as one HIP graph and replayed "
                         "(how a serving loop drives the decode step); host: every GEMV launched from Python")
    ap.add_argument("--no-config5", action="store_true", help="skip the 64-layer sweep and the M=7300 GEMMs")
    ap.add_argument("--no-ffn", action="store_true", help="skip the FFN sublayer figures")
    ap.add_argument("--calib-only", action="store_true",
                    help="only the calibration kernels (launch floor, plain read), then print them and exit")
    ap.add_argument("--gemm-only", action="store_true",
                    help="only the pp512 prefill GEMMs (for counter runs), then exit")
    ap.add_argument("--wide-only", action="store_true",
                    help="only the wide verification GEMV figures (for profiler runs), then exit")
    ap.add_argument("--ffn-only", action="store_true",
                    help="only the FFN sublayer figures (for profiler runs), then exit")
    ap.add_argument("--lm-head-only", action="store_true",
                    help="only the lm_head GEMV, its argmax and its weight-load stream alone, then exit")
    ap.add_argument("--q8-only", action="store_true",
                    help="only the Q8_0 MTP-head GEMV figures (for profiler runs), then exit")
    ap.add_argument("--step-only", action="store_true",
                    help="only the timed decode-sweep steps (for counter runs), then print value and exit")
    ap.add_argument("--reps", type=int, default=200, help="repeats per matrix for the per-matrix tables")
    ap.add_argument("--calib-sweep", action="store_true",
                    help="only the plain-read sweep over geometries (threads, workgroups per CU, loads in "
                         "flight, non-temporal hint) behind the read ceiling, then print it and exit")
    ap.add_argument("--calib-copy", type=int, default=0, metavar="MB",
                    help="only run 20 plain torch copies of MB MiB (HBM-counter calibration) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 "
                                   "(the multi-GPU plan is design-only: decode is replicated, see DESIGN.md)"}))
        sys.exit(2)

    import torch
    from kata_amd import ops

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream(dev)
    if args.calib_only:
        print(json.dumps({"calibration": run_calibration(torch, ops, dev, stream, torch.cuda.Stream(dev), args.reps)}))
        return

    if args.calib_sweep:
        print(json.dumps({"calib_sweep": run_calib_sweep(torch, ops, dev, stream, torch.cuda.Stream(dev))}))
        return

    if args.calib_copy:
        # a plain device copy of known size: its FETCH_SIZE / WRITE_SIZE readings give the
        # counters' scale factor for the HBM-traffic figure
        n = args.calib_copy << 20
        src = torch.ones(n, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(20):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calib_copy_bytes": n}))
        return

    # ---- weights: one layer-set per copy, copies until >= 512 MB
    set_bytes = sum(packed_bytes(K, N) for _, K, N, _ in SWEEP)
    ncopies = max(2, -(-512 * 1024 * 1024 // set_bytes))
    base = [make_weights(torch, dev, K, N, SEED + i, ops) for i, (_, K, N, _) in enumerate(SWEEP)]
    copies = [base] + [[w.clone() for w in base] for _ in range(ncopies - 1)]
    xs = {}
    for gi, grp in enumerate(sorted({g for *_, g in SWEEP})):
        K = next(K for _, K, _, g in SWEEP if g == grp)
        xs[grp] = torch.from_numpy(np.random.default_rng(SEED + 77 + gi).standard_normal((1, K))
                                   .astype(np.float16)).to(dev)
    ys = [torch.empty((1, N), dtype=torch.float32, device=dev) for _, _, N, _ in SWEEP]
    # the operand form of each input (what the input transform writes in the decode path)
    xqs = {grp: ops.gemv_prepare_x(x, x.shape[1], 1) for grp, x in xs.items()}

    if args.gemm_only:
        print(json.dumps({"prefill_gemm": run_gemm(torch, ops, dev, stream, copies, ncopies)}))
        return
    if args.ffn_only:
        cs = torch.cuda.Stream(dev)
        print(json.dumps({"ffn_sublayer": run_ffn(torch, ops, dev, stream,
                                                  lambda fn, n: graph_time(torch, fn, n, stream, cs))}))
        return
    if args.lm_head_only:
        cs = torch.cuda.Stream(dev)
        print(json.dumps({"lm_head": run_lm_head(torch, ops, dev, xqs[next(g for _, K, _, g in SWEEP if K == 5120)],
                                                 lambda fn, n: graph_time(torch, fn, n, stream, cs))}))
        return
    if args.q8_only:
        cs = torch.cuda.Stream(dev)
        print(json.dumps({"q8_0_t1": run_q8(torch, ops, dev, lambda fn, n: graph_time(torch, fn, n, stream, cs),
                                            args.reps)}))
        return
    if args.wide_only:
        cs = torch.cuda.Stream(dev)
        print(json.dumps({"verify_wide": run_verify_wide(torch, ops, dev, copies, ncopies,
                                                         lambda fn, n: graph_time(torch, fn, n, stream, cs), args.reps)}))
        return

    groups = {}
    for j, (name, K, N, grp) in enumerate(SWEEP):
        groups.setdefault(grp, []).append(j)
    group_list = [(grp, idx, SWEEP[idx[0]][1]) for grp, idx in groups.items()]

    def step(i, xin=xqs):
        ws = copies[i % ncopies]
        for grp, idx, K in group_list:
            ops.gemv_ptq1_batch([ws[j] for j in idx], xin[grp], K, [SWEEP[j][2] for j in idx], 1,
                                outs=[ys[j] for j in idx])

    def step_raw(i):
        step(i, xs)

    def step_single(i):
        ws = copies[i % ncopies]
        for j, (name, K, N, grp) in enumerate(SWEEP):
            ops.gemv_ptq1(ws[j], xqs[grp], K, N, 1, out=ys[j])

    # The timed steps run either as captured HIP graphs (default: a batch of consecutive steps
    # per graph, step i on weight copy i % ncopies, captured before the timed region and
    # replayed inside it) or as host launches from Python, one call per GEMV launch.
    cap_stream = torch.cuda.Stream(dev)            # capture needs a non-default stream
    fns = {"step": step} if args.step_only else {"step": step, "single": step_single, "raw": step_raw}
    for fn in fns.values():
        for i in range(2):
            fn(i)                                 # first calls set kernel attributes
    torch.cuda.synchronize()

    batch_ms = []

    def timed(fname, n_steps, nbatch=1, launch=args.launch):
        """ms of n_steps steps; with nbatch > 1 also events between nbatch equal batches of
        them (batch_ms), for the best / median batch figures."""
        fn = fns[fname]
        cuts = [(b * n_steps) // nbatch for b in range(nbatch + 1)]
        graphs = []
        if launch == "graph":
            for b in range(nbatch):
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g, stream=cap_stream):
                    for i in range(cuts[b], cuts[b + 1]):
                        fn(i)
                graphs.append(g)
            for g in graphs:                      # a first replay uploads each graph (untimed)
                g.replay()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(nbatch + 1)]
        torch.cuda.synchronize()
        def run_all():
            for b in range(nbatch):
                if launch == "graph":
                    graphs[b].replay()
                else:
                    for i in range(cuts[b], cuts[b + 1]):
                        fn(i)
        # untimed: the same steps back to back for >= WARM_MS, then the timed ones with no
        # host synchronisation in between (the clock drops while the GPU idles)
        w0, w1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        w0.record(stream)
        run_all()
        w1.record(stream)
        torch.cuda.synchronize()
        for _ in range(math.ceil(WARM_MS / max(w0.elapsed_time(w1), 1e-3))):
            run_all()
        ev[0].record(stream)
        for b in range(nbatch):
            if launch == "graph":
                graphs[b].replay()
            else:
                for i in range(cuts[b], cuts[b + 1]):
                    fn(i)
            ev[b + 1].record(stream)
        torch.cuda.synchronize()
        if nbatch > 1:
            batch_ms[:] = [ev[j].elapsed_time(ev[j + 1]) / max(1, cuts[j + 1] - cuts[j]) for j in range(nbatch)]
        return ev[0].elapsed_time(ev[nbatch])

    for i in range(args.warmup):
        fns["step"](i)
    torch.cuda.synchronize()
    nbatch = 8 if args.steps >= 8 else 1
    ms_total = timed("step", args.steps, nbatch=nbatch)
    step_batch_ms = list(batch_ms)
    ms_step = ms_total / args.steps
    value = set_bytes * args.steps / (ms_total * 1e-3) / 1e9
    if args.step_only:
        print(json.dumps({"value": round(value, 1), "unit": "GB/s", "ms_per_step": round(ms_step, 5)}))
        return

    # ---- dominant kernel: a step is nothing but its GEMV launches
    launches = len(group_list)
    gemv_launch_us = ms_total * 1e3 / (args.steps * launches)
    ms_single = timed("single", args.steps)
    ms_raw = timed("raw", args.steps, nbatch=nbatch)      # batched as the headline step
    other = "host" if args.launch == "graph" else "graph"
    ms_other = timed("step", args.steps, launch=other)
    bytes_per_launch = set_bytes / launches
    achieved = bytes_per_launch / (gemv_launch_us * 1e-6) / 1e9

    # ---- per matrix kind (config 2: 200 repeats each over rotating copies)
    per_matrix = {}
    def time_reps(fn, nrep):
        return graph_time(torch, fn, nrep, stream, cap_stream)

    for j, (name, K, N, grp) in enumerate(SWEEP):
        us = time_reps(lambda r: ops.gemv_ptq1(copies[r % ncopies][j], xqs[grp], K, N, 1, out=ys[j]), args.reps)
        us_raw = time_reps(lambda r: ops.gemv_ptq1(copies[r % ncopies][j], xs[grp], K, N, 1, out=ys[j]), args.reps)
        per_matrix[name] = {"K": K, "N": N, "us": round(us, 3),
                            "GBps": round(packed_bytes(K, N) / (us * 1e-6) / 1e9, 1), "raw_x_us": round(us_raw, 3)}

    calib = run_calibration(torch, ops, dev, stream, cap_stream, args.reps)
    calib["ffn_gate_vs_read_19.5MB"] = round(per_matrix["ffn_gate"]["us"] / calib["19.5MB"]["us"], 3)
    calib["ffn_gate_vs_ceiling_19.5MB"] = round(per_matrix["ffn_gate"]["us"] / calib["19.5MB"]["peak_us"], 3)
    # the GEMV's own weight-load stream alone (its loads, order and ring; nothing else)
    jgate = next(j for j, s_ in enumerate(SWEEP) if s_[0] == "ffn_gate")
    cw = torch.zeros(4, dtype=torch.int32, device=dev)
    us_ws = time_reps(lambda r: ops.calib_read_ptq1(copies[r % ncopies][jgate], 5120, 17408, cw), args.reps)
    calib["ffn_gate_weight_stream_us"] = round(us_ws, 3)
    calib["ffn_gate_vs_weight_stream"] = round(per_matrix["ffn_gate"]["us"] / us_ws, 3)

    # ---- config 3: T=2 speculative-verify GEMV (two fp16 activation columns
    # shared per input) and the Q8_0 MTP-head GEMV (17408x5120 and 5120x17408, T=1)
    verify_t2 = {}
    for j, (name, K, N, grp) in enumerate(SWEEP):
        if name not in ("gdn_qkv", "attn_q", "attn_o", "ffn_gate", "ffn_down"):
            continue
        x2 = torch.from_numpy(np.random.default_rng(SEED + 300 + j).standard_normal((2, K))
                              .astype(np.float16)).to(dev)
        y2 = torch.empty((2, N), dtype=torch.float32, device=dev)
        xq2 = ops.gemv_prepare_x(x2, K, 2)
        us = time_reps(lambda r: ops.gemv_ptq1(copies[r % ncopies][j], xq2, K, N, 2, out=y2), args.reps)
        us_raw = time_reps(lambda r: ops.gemv_ptq1(copies[r % ncopies][j], x2, K, N, 2, out=y2), args.reps)
        verify_t2[name] = {"K": K, "N": N, "us": round(us, 3),
                           "GBps": round(packed_bytes(K, N) / (us * 1e-6) / 1e9, 1), "raw_x_us": round(us_raw, 3)}
    verify_wide = run_verify_wide(torch, ops, dev, copies, ncopies,
                                  lambda fn, n: graph_time(torch, fn, n, stream, cap_stream), args.reps)
    q8 = run_q8(torch, ops, dev, time_reps, args.reps)

    # ---- lm_head (5120 -> 248320 PTQ1_0 GEMV, 278 MB) and the greedy argmax of its logits
    lm_head = run_lm_head(torch, ops, dev, xqs[next(g for _, K, _, g in SWEEP if K == 5120)], time_reps)

    # ---- matmul input transform (residual add + RMSNorm + sign + FWHT), decode and prefill
    xform = {}
    for label, M, odt in (("decode_m1", 1, 1), ("decode_m1_operand", 1, 2), ("prefill_m7300", 7300, 1)):
        W = 5120
        xt = torch.randn((M, W), device=dev)
        yt = torch.randn((M, W), device=dev)
        gt = torch.sign(torch.randn(W, device=dev))
        obytes = ops.gemv_xq_bytes(W, M) if odt == 2 else M * W * 2
        outt = torch.empty(obytes, dtype=torch.uint8, device=dev)
        xn = torch.empty_like(xt)

        def xf(r, xt=xt, yt=yt, gt=gt, outt=outt, xn=xn, W=W, M=M, odt=odt):
            ops.check(ops.lib().kata_add_rms_fwht(ops._ptr(xt), ops._ptr(yt), ops._ptr(gt), ops._ptr(outt), odt, 0,
                                                  ops._ptr(xn), None, None, 0, W, M, ops._stream(xt)))
        us = time_reps(xf, 50 if M > 1 else args.reps)
        nbytes = M * W * (4 + 4 + 4) + obytes          # x, y in; xnew fp32 and out (fp16 / operand) out
        xform[label] = {"M": M, "W": W, "out": "operand form" if odt == 2 else "fp16 rows", "us": round(us, 2),
                        "GBps": round(nbytes / (us * 1e-6) / 1e9, 1)}

    # ---- layer level: the FFN sublayer (27B shapes) through the dispatcher
    ffn = None if args.no_ffn else run_ffn(torch, ops, dev, stream, time_reps)

    # ---- pp512 prefill GEMM (config 4), fp16 exact path
    gemm = None if args.no_gemm else run_gemm(torch, ops, dev, stream, copies, ncopies)

    # ---- config 5: full 64-layer decode pass, M=7300 prefill
    cfg5 = None
    if not args.no_config5:
        cfg5 = run_config5(torch, ops, dev, stream)

    # ---- CPU baseline (reference host arithmetic, bounded sample)
    cpu = None
    if not args.no_cpu:
        # all cores this process may use: the CPU affinity set, capped by the harness's per-GPU
        # CPU share when one is set (OMP_NUM_THREADS)
        nproc = os.cpu_count() or 1
        avail = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else nproc
        share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
        threads = min(avail, share) if share > 0 else avail
        gbs, nbytes = cpu_baseline(threads)
        gbs1, _ = cpu_baseline(1, reps=1)
        cpu = {"value": round(gbs, 3), "unit": "GB/s", "cores": threads, "kind": "port",
               "sample": f"BASELINE config 1 in full: 17408x5120 PTQ1_0 ({nbytes/1e6:.1f} MB packed), one fp32 "
                         f"activation; stage-loop row dequantisation (dequantize_row_ptq1_0) + fp32 dot, "
                         f"OpenMP over rows, best of 3; nproc={nproc}, affinity={avail}, "
                         f"OMP_NUM_THREADS={share or 'unset'}",
               "single_thread": {"value": round(gbs1, 3), "unit": "GB/s", "cores": 1,
                                 "sample": "the same full matrix, one thread"},
               "prefill_gemm": cpu_gemm_baseline(threads)}

    # HBM bytes per launch of the dominant kernel, from the committed rocprofv3 PMC summary
    traffic = None
    tpath = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "gemv_ptq1_decode_sweep.md")
    if os.path.exists(tpath):
        with open(tpath) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    traffic = int(line.split(":")[1])

    out = {
        "metric": "ternary GEMV HBM GB/s (% of peak) at bs=1; pp512 prefill GEMM TFLOPS",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16 in -> 16-bit block fixed point (2 x int8 limbs) x int8 trits -> exact int32 -> fp32 out",
        "numerics": ("fp16 activation -> per-128-block 16-bit fixed point as two int8 limbs; ternary weights as "
                     "int8 trits; exact int32 block sums on the int8 matrix cores; fp32 scale (fp16 d x block "
                     "scale) and fp32 accumulation; fp32 output"),
        "data": "synthetic (seeded trits/scales/activations)",
        "config": {"workload": "BASELINE configs[1]: bs=1 decode GEMV sweep, one layer of each kind "
                               "(10 matrices in 6 launches, matrices sharing an input batched)",
                   "weight_copies": ncopies, "bytes_per_step": set_bytes, "launch": args.launch},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": "k_gemv_ptq1<1>", "avg_launch_us": round(gemv_launch_us, 3),
                     "bytes_per_launch": bytes_per_launch},
        "step_batches": ({"n": len(step_batch_ms),
                          "best_GBps": round(set_bytes / (min(step_batch_ms) * 1e-3) / 1e9, 1),
                          "median_GBps": round(set_bytes / (float(np.median(step_batch_ms)) * 1e-3) / 1e9, 1)}
                         if step_batch_ms else None),
        f"{other}_launch": {"ms_per_step": round(ms_other / args.steps, 5),
                            "GBps": round(set_bytes * args.steps / (ms_other * 1e-3) / 1e9, 1)},
        "raw_x_step": {"ms_per_step": round(ms_raw / args.steps, 5),
                       "GBps": round(set_bytes * args.steps / (ms_raw * 1e-3) / 1e9, 1),
                       "note": "the same step on fp16 rows, quantised by every GEMV workgroup"},
        "one_launch_per_matrix": {"ms_per_step": round(ms_single / args.steps, 5),
                                  "GBps": round(set_bytes * args.steps / (ms_single * 1e-3) / 1e9, 1)},
        "per_matrix": per_matrix,
        "calibration": calib,
        "verify_t2": verify_t2,
        "verify_wide": verify_wide,
        "q8_0_t1": q8,
        "prefill_gemm": gemm,
        "input_transform": xform,
        "lm_head": lm_head,
        "ffn_sublayer": ffn,
        "config5": cfg5,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
