"""Writes tests/golden/ptq1_golden.npz: small known-answer vectors for the ternary path.

The reference repository commits no numeric fixtures for this path, so these vectors are
computed here from first principles, in plain Python integers and float64, with code that
shares nothing with oracle/kata_oracle.c:

* digits from the base-3 fraction definition: digit n of byte b is
  floor(b * 3^(n+1) / 256) mod 3 (the packed byte is ceil(q*256/243) for the 5-digit
  base-3 number q, docs/reference/prism_ptq1_0_quant_dequant.c:30-31), not the
  ((b*3^n mod 256)*3)>>8 form the oracle and the kernels use;
* the element map from its prose statement in docs/MODEL_SPEC.en.md:101-103;
* packing from the quantiser definition (prism_ptq1_0_quant_dequant.c:20-46) with exact
  integer ceil division;
* GEMV / GEMM sums in float64 over Python lists; quant_rows in float32 numpy scalars
  (IEEE ops, as shaders/prefill.metal:373-377); int8 group sums in Python integers.

Run:  python tests/golden/make_golden.py   (deterministic: fixed seeds)
"""
from __future__ import annotations

import os

import numpy as np

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "ptq1_golden.npz")


def digit_def(b: int, n: int) -> int:
    return (b * 3 ** (n + 1) // 256) % 3


def elem_source(e: int):
    """(byte, digit) holding element e of a 128-element block (MODEL_SPEC 7)."""
    if e < 80:
        return e % 16, e // 16          # n-th trit of qs[m] -> element n*16+m
    if e < 120:
        return 16 + (e - 80) % 8, (e - 80) // 8   # qs[16+m] -> 80+n*8+m
    return 24 + (e - 120) % 2, (e - 120) // 2     # qh[h] -> 120+n*2+h


def pack_block(trits, d_f16: np.float16) -> bytes:
    blk = [0] * 28
    for p in range(26):
        nd = 5 if p < 24 else 4
        q = 0
        for n in range(nd):
            # element holding (p, n)
            if p < 16:
                e = 16 * n + p
            elif p < 24:
                e = 80 + 8 * n + (p - 16)
            else:
                e = 120 + 2 * n + (p - 24)
            q = 3 * q + (int(trits[e]) + 1)
        if nd == 4:
            q *= 3
        blk[p] = -((-q * 256) // 243)   # ceil(q*256/243)
    raw = np.array([d_f16], dtype=np.float16).view(np.uint8)
    blk[26], blk[27] = int(raw[0]), int(raw[1])
    return bytes(blk)


def decode_block(blk: bytes):
    d = float(np.frombuffer(blk[26:28], dtype=np.float16)[0])
    out = []
    for e in range(128):
        p, n = elem_source(e)
        out.append(digit_def(blk[p], n) - 1)
    return out, d


def main():
    rng = np.random.default_rng(20260101)
    g = {}
    # 1. exhaustive digit table
    g["digit_table"] = np.array([[digit_def(b, n) for n in range(5)] for b in range(256)], np.int8)
    g["elem_byte"] = np.array([elem_source(e)[0] for e in range(128)], np.int16)
    g["elem_digit"] = np.array([elem_source(e)[1] for e in range(128)], np.int16)

    # 2. a small PTQ1_0 matrix: N=24 rows, K=256 (2 blocks); trits + scales -> bytes
    N, K = 24, 256
    trits = rng.integers(-1, 2, size=(N, K)).astype(np.int8)
    scales = np.abs(rng.normal(0, 0.02, size=(N, K // 128))).astype(np.float16)
    scales[3, 1] = np.float16(0.0)                          # d = 0 block
    trits[5, :] = 0                                          # all-zero row
    trits[7, :] = 0; trits[7, 123] = 1                       # single hot element (qh area)
    trits[8, :] = 0; trits[8, 87] = -1                       # single hot element (c=8 stage)
    W = b"".join(pack_block(list(trits[n, 128 * b:128 * b + 128]), scales[n, b])
                 for n in range(N) for b in range(K // 128))
    W = np.frombuffer(W, np.uint8).reshape(N, K // 128 * 28).copy()
    g["ptq1_W"], g["ptq1_trits"], g["ptq1_scales"] = W, trits, scales
    g["ptq1_K"], g["ptq1_N"] = np.int32(K), np.int32(N)

    # dequantised values from the independent decoder
    deq = np.zeros((N, K), np.float64)
    for n in range(N):
        for b in range(K // 128):
            t, d = decode_block(W[n, b * 28:(b + 1) * 28].tobytes())
            for e in range(128):
                deq[n, 128 * b + e] = t[e] * d
    g["ptq1_deq"] = deq

    # 3. GEMV T=1 and T=2 with fp16 activations (values widened exactly)
    x = rng.standard_normal((2, K)).astype(np.float16)
    x[1, :] = np.float16(1.0)                                # x = 1 -> d * sum(t)
    g["gemv_x"] = x
    xf = x.astype(np.float64)
    y = np.zeros((2, N))
    for t in range(2):
        for n in range(N):
            s = 0.0
            for k in range(K):
                s += deq[n, k] * xf[t, k]
            y[t, n] = s
    g["gemv_y"] = y

    # 4. Q8_0: N=8, K=64
    Nq, Kq = 8, 64
    q = rng.integers(-127, 128, size=(Nq, Kq)).astype(np.int8)
    qs = np.abs(rng.normal(0, 0.02, size=(Nq, Kq // 32))).astype(np.float16)
    Wq = np.zeros((Nq, Kq // 32, 34), np.uint8)
    Wq[:, :, 0:2] = qs.view(np.uint8).reshape(Nq, Kq // 32, 2)
    Wq[:, :, 2:] = q.view(np.uint8).reshape(Nq, Kq // 32, 32)
    xq = rng.standard_normal((2, Kq)).astype(np.float16)
    yq = np.zeros((2, Nq))
    for t in range(2):
        for n in range(Nq):
            acc = 0.0
            for b in range(Kq // 32):
                s = sum(int(q[n, 32 * b + i]) * float(xq[t, 32 * b + i]) for i in range(32))
                acc += float(qs[n, b]) * s
            yq[t, n] = acc
    g["q8_W"], g["q8_x"], g["q8_y"] = Wq.reshape(Nq, -1), xq, yq

    # 5. fp16 GEMM M=5 (ragged), on the PTQ1_0 matrix above
    M = 5
    A = rng.standard_normal((M, K)).astype(np.float16)
    wexp = deq.astype(np.float16)                           # exact: t*d is an fp16 value
    assert np.array_equal(wexp.astype(np.float64), deq)
    C = np.zeros((M, N))
    for m in range(M):
        for n in range(N):
            C[m, n] = sum(float(A[m, k]) * float(wexp[n, k]) for k in range(K))
    g["gemm_A"], g["gemm_C"], g["expand_f16"] = A, C, wexp

    # 6. quant_rows on A (float32 scalar IEEE arithmetic), incl. an all-zero group and a tie
    Xr = rng.standard_normal((3, K)).astype(np.float16)
    Xr[1, 128:] = np.float16(0.0)
    Xr[2, 0] = np.float16(127.0); Xr[2, 1] = np.float16(0.5); Xr[2, 2] = np.float16(1.5); Xr[2, 3] = np.float16(-2.5)
    Xr[2, 4:128] = np.float16(0.0)
    Qr = np.zeros((3, K), np.int8)
    SXr = np.zeros((K // 128, 3), np.float32)
    for m in range(3):
        for gi in range(K // 128):
            v = Xr[m, 128 * gi:128 * gi + 128].astype(np.float32)
            mx = np.float32(0.0)
            for a in v:
                mx = max(mx, np.float32(abs(a)))
            scale = np.float32(mx / np.float32(127.0)) if mx > 0 else np.float32(1.0)
            inv = np.float32(np.float32(1.0) / scale)
            for i in range(128):
                r = np.float32(np.rint(np.float32(v[i] * inv)))
                Qr[m, 128 * gi + i] = int(min(max(r, -127.0), 127.0))
            SXr[gi, m] = scale
    g["qr_X"], g["qr_Q"], g["qr_SX"] = Xr, Qr, SXr

    # 7. int8 GEMM group sums on (Qr, trits of the PTQ1_0 matrix)
    GS = np.zeros((3, N, K // 128), np.int64)
    for m in range(3):
        for n in range(N):
            for gi in range(K // 128):
                GS[m, n, gi] = sum(int(Qr[m, 128 * gi + i]) * int(trits[n, 128 * gi + i]) for i in range(128))
    g["i8_GS"] = GS.astype(np.int32)

    np.savez(OUT, **g)
    print("wrote", OUT, {k: v.shape for k, v in g.items()})


if __name__ == "__main__":
    main()
