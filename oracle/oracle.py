"""ctypes front end of the CPU oracle (oracle/kata_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, always as the checker or the timed CPU baseline.  The product path
(kata_amd/) never imports this module.

Also holds the seeded synthetic-data generators for the BASELINE configurations
(trits iid uniform on {-1,0,+1}, fp16 scales |N(0,0.02)|, fp16 N(0,1) activations,
Q8_0 int8 uniform in [-127,127]).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "_build", "liboracle.so")
_lib = None

GROUP = 128
BLOCK_BYTES = 28
Q8_GROUP = 32
Q8_BLOCK_BYTES = 34


def build() -> str:
    subprocess.run(["make", "-C", _HERE, "-s"], check=True)
    return _SO


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_SO):
            build()
        L = ctypes.CDLL(_SO)
        P = ctypes.c_void_p
        i, i64 = ctypes.c_int, ctypes.c_int64
        sig = {
            "orc_half_to_float": (ctypes.c_float, [ctypes.c_uint16]),
            "orc_float_to_half": (ctypes.c_uint16, [ctypes.c_float]),
            "orc_ptq1_digit": (i, [ctypes.c_uint32, ctypes.c_uint32]),
            "orc_ptq1_digit_float": (i, [ctypes.c_uint32, ctypes.c_uint32]),
            "orc_ptq1_elem_trit": (i, [P, i]),
            "orc_ptq1_dequant_row": (None, [P, P, i64]),
            "orc_ptq1_quant_row": (None, [P, P, i64]),
            "orc_ptq1_pack_row": (None, [P, P, P, i64]),
            "orc_gemv_ptq1": (None, [P, P, P, i, i, i]),
            "orc_gemv_q8": (None, [P, P, P, i, i, i]),
            "orc_expand_ptq1_f16": (None, [P, P, i, i]),
            "orc_gemm_ptq1_f16": (None, [P, P, P, i, i, i]),
            "orc_quant_rows": (None, [P, P, P, i, i, i]),
            "orc_expand_ptq1_i8": (None, [P, P, P, i, i]),
            "orc_gemm_i8": (None, [P, P, i, P, P, P, i, i, i]),
            "orc_cpu_gemv_ptq1_f32": (None, [P, P, P, i, i, i, i, i, i]),
            "orc_expand_q8_f16": (None, [P, P, i, i]),
            "orc_gemm_q8_f16": (None, [P, P, P, i, i, i]),
            "orc_cpu_gemv_ptq1_stage": (None, [P, P, P, i, i, i, i, i, i]),
            "orc_cpu_gemm_ptq1_f32": (None, [P, P, P, i, i, i, i, i, i]),
            "orc_norm_fwht": (None, [P, P, P, P, P, P, i, i, i, i]),
            "orc_omp_max_threads": (i, []),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype, f.argtypes = res, args
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


# ----------------------------------------------------------------------------- PTQ1_0
def digit(b: int, n: int) -> int:
    return lib().orc_ptq1_digit(b, n)


def dequant(W: np.ndarray, K: int, N: int) -> np.ndarray:
    """PTQ1_0 [N][K/128 blocks] -> float32 [N][K] (dequantize_row_ptq1_0)."""
    W = np.ascontiguousarray(W, dtype=np.uint8).reshape(N, K // GROUP * BLOCK_BYTES)
    out = np.empty((N, K), np.float32)
    for n in range(N):
        lib().orc_ptq1_dequant_row(_p(W[n]), _p(out[n]), K)
    return out


def quantize(X: np.ndarray) -> np.ndarray:
    """float32 [N][K] -> PTQ1_0 bytes [N][K/128*28] (quantize_row_ptq1_0_ref)."""
    X = np.ascontiguousarray(X, dtype=np.float32)
    N, K = X.shape
    out = np.empty((N, K // GROUP * BLOCK_BYTES), np.uint8)
    for n in range(N):
        lib().orc_ptq1_quant_row(_p(X[n]), _p(out[n]), K)
    return out


def pack(trits: np.ndarray, scales_f16: np.ndarray) -> np.ndarray:
    """int8 trits [N][K] + fp16 scales [N][K/128] -> PTQ1_0 bytes [N][K/128*28]."""
    trits = np.ascontiguousarray(trits, dtype=np.int8)
    N, K = trits.shape
    sc = np.ascontiguousarray(scales_f16, dtype=np.float16).view(np.uint16).reshape(N, K // GROUP)
    out = np.empty((N, K // GROUP * BLOCK_BYTES), np.uint8)
    for n in range(N):
        lib().orc_ptq1_pack_row(_p(trits[n]), _p(np.ascontiguousarray(sc[n])), _p(out[n]), K)
    return out


def gemv_ptq1(W, x, K, N, T) -> np.ndarray:
    """fp64 oracle: y[T][N] for x[T][K] (float32 view of the activations)."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(T, K)
    W = np.ascontiguousarray(W, dtype=np.uint8)
    y = np.empty((T, N), np.float64)
    lib().orc_gemv_ptq1(_p(W), _p(x), _p(y), K, N, T)
    return y


def gemv_q8(W, x, K, N, T) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(T, K)
    W = np.ascontiguousarray(W, dtype=np.uint8)
    y = np.empty((T, N), np.float64)
    lib().orc_gemv_q8(_p(W), _p(x), _p(y), K, N, T)
    return y


def expand_f16(W, K, N) -> np.ndarray:
    W = np.ascontiguousarray(W, dtype=np.uint8)
    out = np.empty((N, K), np.uint16)
    lib().orc_expand_ptq1_f16(_p(W), _p(out), K, N)
    return out.view(np.float16)


def gemm_f16(A, W, M, K, N) -> np.ndarray:
    A = np.ascontiguousarray(A, dtype=np.float16).view(np.uint16)
    W = np.ascontiguousarray(W, dtype=np.uint8)
    C = np.empty((M, N), np.float64)
    lib().orc_gemm_ptq1_f16(_p(A), _p(W), _p(C), M, K, N)
    return C


def expand_q8_f16(W, K, N) -> np.ndarray:
    """k_expand_q8: fp16 half(d * q) of every Q8_0 element, [N][K]."""
    W = np.ascontiguousarray(W, dtype=np.uint8)
    out = np.empty((N, K), np.uint16)
    lib().orc_expand_q8_f16(_p(W), _p(out), K, N)
    return out.view(np.float16)


def gemm_q8_f16(A, W, M, K, N) -> np.ndarray:
    """MTP K/V catch-up GEMM: A fp16 [M][K] times the expanded Q8_0 matrix, double sums."""
    A = np.ascontiguousarray(A, dtype=np.float16).view(np.uint16)
    W = np.ascontiguousarray(W, dtype=np.uint8)
    C = np.empty((M, N), np.float64)
    lib().orc_gemm_q8_f16(_p(A), _p(W), _p(C), M, K, N)
    return C


def quant_rows(X, M, K, ldS=None):
    ldS = M if ldS is None else ldS
    X = np.ascontiguousarray(X, dtype=np.float16).view(np.uint16)
    Q = np.empty((M, K), np.int8)
    SX = np.zeros((K // GROUP, ldS), np.float32)
    lib().orc_quant_rows(_p(X), _p(Q), _p(SX), M, K, ldS)
    return Q, SX


def expand_i8(W, K, N):
    W = np.ascontiguousarray(W, dtype=np.uint8)
    T8 = np.empty((N, K), np.int8)
    SW = np.empty((N, K // GROUP), np.float32)
    lib().orc_expand_ptq1_i8(_p(W), _p(T8), _p(SW), K, N)
    return T8, SW


def gemm_i8(A8, SX, W, M, K, N, want_group_sums=False):
    A8 = np.ascontiguousarray(A8, dtype=np.int8)
    SX = np.ascontiguousarray(SX, dtype=np.float32)
    ldS = SX.shape[1]
    W = np.ascontiguousarray(W, dtype=np.uint8)
    C = np.empty((M, N), np.float32)
    GS = np.empty((M, N, K // GROUP), np.int32) if want_group_sums else None
    lib().orc_gemm_i8(_p(A8), _p(SX), ldS, _p(W), _p(C), _p(GS) if GS is not None else None, M, K, N)
    return (C, GS) if want_group_sums else C


def norm_fwht(src, gs, mode, src2=None, gamma=None, add=False):
    """Input transform (double): returns (out [M][W], hout or None)."""
    src = np.ascontiguousarray(src, dtype=np.float32)
    M, W = src.shape
    gs = np.ascontiguousarray(gs, dtype=np.float32)
    s2 = None if src2 is None else np.ascontiguousarray(src2, dtype=np.float32)
    gm = None if gamma is None else np.ascontiguousarray(gamma, dtype=np.float32)
    out = np.empty((M, W), np.float64)
    hout = np.empty((M, W), np.float64) if gm is not None else None
    lib().orc_norm_fwht(_p(src), None if s2 is None else _p(s2), _p(gs), None if gm is None else _p(gm), _p(out),
                        None if hout is None else _p(hout), W, M, mode, 1 if add else 0)
    return out, hout


def cpu_gemm_f32(A, W, M, K, N, row0, nrows, nthreads):
    """CPU baseline GEMM (fp32) over weight rows [row0, row0 + nrows); C is [M][N]."""
    A = np.ascontiguousarray(A, dtype=np.float16).view(np.uint16)
    W = np.ascontiguousarray(W, dtype=np.uint8)
    C = np.zeros((M, N), np.float32)
    lib().orc_cpu_gemm_ptq1_f32(_p(A), _p(W), _p(C), M, K, N, row0, nrows, nthreads)
    return C


def cpu_gemv_stage(W, x, K, N, T, row0, nrows, nthreads):
    """CPU baseline in the reference's host form: stage-loop row dequantisation + fp32 dot."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(T, K)
    W = np.ascontiguousarray(W, dtype=np.uint8)
    y = np.zeros((T, N), np.float32)
    lib().orc_cpu_gemv_ptq1_stage(_p(W), _p(x), _p(y), K, N, T, row0, nrows, nthreads)
    return y


def cpu_gemv_f32(W, x, K, N, T, row0, nrows, nthreads):
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(T, K)
    W = np.ascontiguousarray(W, dtype=np.uint8)
    y = np.zeros((T, N), np.float32)
    lib().orc_cpu_gemv_ptq1_f32(_p(W), _p(x), _p(y), K, N, T, row0, nrows, nthreads)
    return y


# ----------------------------------------------------------------------------- Q8_0
def q8_pack(q: np.ndarray, scales_f16: np.ndarray) -> np.ndarray:
    """int8 [N][K] + fp16 [N][K/32] -> Q8_0 bytes [N][K/32*34]."""
    N, K = q.shape
    nb = K // Q8_GROUP
    out = np.empty((N, nb, Q8_BLOCK_BYTES), np.uint8)
    out[:, :, 0:2] = np.ascontiguousarray(scales_f16, np.float16).view(np.uint8).reshape(N, nb, 2)
    out[:, :, 2:] = np.ascontiguousarray(q, np.int8).view(np.uint8).reshape(N, nb, Q8_GROUP)
    return out.reshape(N, nb * Q8_BLOCK_BYTES)


# ----------------------------------------------------------------------------- synthetic data
def synth_ptq1(N: int, K: int, seed: int):
    """Trits iid uniform on {-1,0,+1}; scales fp16(|N(0,0.02)|) per 128-group; packed."""
    rng = np.random.default_rng(seed)
    trits = rng.integers(-1, 2, size=(N, K), dtype=np.int8)
    scales = np.abs(rng.normal(0.0, 0.02, size=(N, K // GROUP))).astype(np.float16)
    return pack(trits, scales), trits, scales


def synth_q8(N: int, K: int, seed: int):
    rng = np.random.default_rng(seed)
    q = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
    scales = np.abs(rng.normal(0.0, 0.02, size=(N, K // Q8_GROUP))).astype(np.float16)
    return q8_pack(q, scales), q, scales


def synth_x(T: int, K: int, seed: int, dtype=np.float16):
    rng = np.random.default_rng(seed)
    return rng.standard_normal((T, K)).astype(dtype)
