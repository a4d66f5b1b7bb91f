"""Torch-tensor front end of the C ABI (device memory and streams come from PyTorch; the
arithmetic is the HIP library's).  Every op runs on the tensor's device, on torch's
current stream, and raises KataError on a bad argument — there is no CPU fallback.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from .capi import KATA_F16, KATA_F32, KATA_X_HALF2, KATA_X_ROWS, KATA_XQ, check, lib

GROUP, BLOCK_BYTES = 128, 28
Q8_GROUP, Q8_BLOCK_BYTES = 32, 34


def _ptr(t: torch.Tensor | None):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _stream(t: torch.Tensor):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _need_gpu(*ts: torch.Tensor):
    for t in ts:
        if not t.is_cuda:
            raise ValueError("kata_amd ops take device tensors (no CPU path)")
        if not t.is_contiguous():
            raise ValueError("kata_amd ops take contiguous tensors")


def _bytes(t: torch.Tensor) -> int:
    return t.numel() * t.element_size()


def _need_bytes(name: str, t: torch.Tensor | None, nbytes: int):
    """The kernels read or write nbytes of t from its start: a shorter tensor would be an
    out-of-bounds device access, so it is a ValueError here."""
    if t is not None and _bytes(t) < nbytes:
        raise ValueError(f"{name} holds {_bytes(t)} bytes, the call needs {nbytes}")


def _ptq1_bytes(K: int, N: int) -> int:
    if K <= 0 or K % GROUP or N <= 0:
        raise ValueError(f"K={K} must be a positive multiple of {GROUP}, N={N} positive")
    return N * (K // GROUP) * BLOCK_BYTES


def _xdtype(x: torch.Tensor) -> int:
    if x.dtype == torch.uint8:
        return KATA_XQ
    if x.dtype == torch.float16:
        return KATA_F16
    if x.dtype == torch.float32:
        return KATA_F32
    raise ValueError(f"activation dtype {x.dtype} not supported (fp16, fp32 or the uint8 operand form)")


def _x_bytes(x: torch.Tensor, K: int, T: int) -> int:
    """Bytes the GEMV reads of x: the operand form's size for uint8, else T*K elements."""
    return gemv_xq_bytes(K, T) if x.dtype == torch.uint8 else T * K * x.element_size()


def gemv_xq_bytes(K: int, T: int) -> int:
    """Bytes of the decode GEMV's operand form of T (1, 2) rows of K (0: unsupported)."""
    return int(lib().kata_gemv_xq_bytes(K, T))


def gemv_prepare_x(x: torch.Tensor, K: int, T: int = 1, half2: bool = False,
                   out: torch.Tensor | None = None) -> torch.Tensor:
    """The decode GEMV's operand form (uint8) of x ([T][K] fp16/fp32, or [K][2] fp16 when half2):
    quantised once, then passed as x to gemv_ptq1 / gemv_ptq1_batch (same y bit for bit)."""
    n = gemv_xq_bytes(K, T)
    if n == 0:
        raise ValueError(f"K={K} T={T}: no operand form")
    _need_bytes("x", x, T * K * x.element_size())
    _need_bytes("out", out, n)
    _need_gpu(x)
    xq = out if out is not None else torch.empty(n, dtype=torch.uint8, device=x.device)
    check(lib().kata_gemv_prepare_x(_ptr(x), _xdtype(x), KATA_X_HALF2 if half2 else KATA_X_ROWS, K, T, _ptr(xq),
                                    _stream(x)))
    return xq


# ----------------------------------------------------------------------------- GEMVs
def gemv_ptq1(W: torch.Tensor, x: torch.Tensor, K: int, N: int, T: int = 1, half2: bool = False,
              out: torch.Tensor | None = None) -> torch.Tensor:
    """y[T][N] fp32 = PTQ1_0 W (N x K) times x ([T][K], or [K][2] fp16 when half2)."""
    _need_bytes("W", W, _ptq1_bytes(K, N))
    _need_bytes("x", x, _x_bytes(x, K, T))
    _need_bytes("out", out, T * N * 4)
    _need_gpu(W, x)
    y = out if out is not None else torch.empty((T, N), dtype=torch.float32, device=W.device)
    check(lib().kata_gemv_ptq1(_ptr(W), _ptr(x), _xdtype(x), KATA_X_HALF2 if half2 else KATA_X_ROWS,
                               _ptr(y), K, N, T, _stream(W)))
    return y


def gemv_ptq1_batch(Ws, x: torch.Tensor, K: int, Ns, T: int = 1, half2: bool = False, outs=None):
    """PTQ1_0 GEMVs of up to 4 matrices sharing the activation x, one launch: returns [y_i]."""
    if len(Ws) != len(Ns) or (outs is not None and len(outs) != len(Ns)):
        raise ValueError("Ws, Ns (and outs) must have the same length")
    for i, (W, N) in enumerate(zip(Ws, Ns)):
        _need_bytes(f"Ws[{i}]", W, _ptq1_bytes(K, N))
        _need_bytes(f"outs[{i}]", outs[i] if outs is not None else None, T * N * 4)
    _need_bytes("x", x, _x_bytes(x, K, T))
    _need_gpu(x, *Ws)
    n = len(Ws)
    ys = outs if outs is not None else [torch.empty((T, N), dtype=torch.float32, device=x.device) for N in Ns]
    Wa = (ctypes.c_void_p * n)(*[W.data_ptr() for W in Ws])
    ya = (ctypes.c_void_p * n)(*[y.data_ptr() for y in ys])
    Na = (ctypes.c_int * n)(*Ns)
    check(lib().kata_gemv_ptq1_batch(n, Wa, ya, Na, _ptr(x), _xdtype(x), KATA_X_HALF2 if half2 else KATA_X_ROWS,
                                     K, T, _stream(x)))
    return ys


def _rows(x: torch.Tensor, T: int | None) -> int:
    """Token rows of an activation: x.shape[0] for rows, the given T for the operand form."""
    if x.dtype == torch.uint8:
        if T is None:
            raise ValueError("the operand form needs T")
        return T
    return x.shape[0]


def gemv_ptq1_wide(W: torch.Tensor, x: torch.Tensor, K: int, N: int, out: torch.Tensor | None = None,
                   T: int | None = None) -> torch.Tensor:
    """Wide verification GEMV: y[T][N] fp32 for x [T][K] (fp16 or fp32, T = x.shape[0] in 1..8)
    or the operand form of T rows (uint8, from gemv_prepare_x or a transform)."""
    T = _rows(x, T)
    _need_bytes("W", W, _ptq1_bytes(K, N))
    _need_bytes("x", x, _x_bytes(x, K, T))
    _need_bytes("out", out, T * N * 4)
    _need_gpu(W, x)
    y = out if out is not None else torch.empty((T, N), dtype=torch.float32, device=W.device)
    check(lib().kata_gemv_ptq1_wide(_ptr(W), _ptr(x), _xdtype(x), _ptr(y), K, N, T, _stream(W)))
    return y


def gemv_ptq1_wide_batch(Ws, x: torch.Tensor, K: int, Ns, outs=None, T: int | None = None):
    """Wide verification GEMVs of up to 4 matrices sharing the token rows x [T][K] (fp16 or
    fp32, T = x.shape[0] in 1..8, or their operand form with T given), one launch: returns
    [y_i], y_i [T][N_i] fp32."""
    T = _rows(x, T)
    if len(Ws) != len(Ns) or (outs is not None and len(outs) != len(Ns)):
        raise ValueError("Ws, Ns (and outs) must have the same length")
    for i, (W, N) in enumerate(zip(Ws, Ns)):
        _need_bytes(f"Ws[{i}]", W, _ptq1_bytes(K, N))
        _need_bytes(f"outs[{i}]", outs[i] if outs is not None else None, T * N * 4)
    _need_bytes("x", x, _x_bytes(x, K, T))
    _need_gpu(x, *Ws)
    n = len(Ws)
    ys = outs if outs is not None else [torch.empty((T, N), dtype=torch.float32, device=x.device) for N in Ns]
    Wa = (ctypes.c_void_p * n)(*[W.data_ptr() for W in Ws])
    ya = (ctypes.c_void_p * n)(*[y.data_ptr() for y in ys])
    Na = (ctypes.c_int * n)(*Ns)
    check(lib().kata_gemv_ptq1_wide_batch(n, Wa, ya, Na, _ptr(x), _xdtype(x), K, T, _stream(x)))
    return ys


def gemv_q8(W: torch.Tensor, x: torch.Tensor, K: int, N: int, T: int = 1,
            out: torch.Tensor | None = None) -> torch.Tensor:
    if K <= 0 or K % Q8_GROUP or N <= 0:
        raise ValueError(f"K={K} must be a positive multiple of {Q8_GROUP}, N={N} positive")
    _need_bytes("W", W, N * (K // Q8_GROUP) * Q8_BLOCK_BYTES)
    _need_bytes("x", x, T * K * x.element_size())
    _need_bytes("out", out, T * N * 4)
    _need_gpu(W, x)
    y = out if out is not None else torch.empty((T, N), dtype=torch.float32, device=W.device)
    check(lib().kata_gemv_q8_0(_ptr(W), _ptr(x), _xdtype(x), _ptr(y), K, N, T, _stream(W)))
    return y


def gemv_q8_batch(Ws, x: torch.Tensor, K: int, Ns, T: int = 1, outs=None):
    """Q8_0 GEMVs of up to 4 matrices sharing the activation x [T][K], one launch: returns [y_i]."""
    if len(Ws) != len(Ns) or (outs is not None and len(outs) != len(Ns)):
        raise ValueError("Ws, Ns (and outs) must have the same length")
    if K <= 0 or K % Q8_GROUP:
        raise ValueError(f"K={K} must be a positive multiple of {Q8_GROUP}")
    for i, (W, N) in enumerate(zip(Ws, Ns)):
        _need_bytes(f"Ws[{i}]", W, N * (K // Q8_GROUP) * Q8_BLOCK_BYTES)
        _need_bytes(f"outs[{i}]", outs[i] if outs is not None else None, T * N * 4)
    _need_bytes("x", x, T * K * x.element_size())
    _need_gpu(x, *Ws)
    n = len(Ws)
    ys = outs if outs is not None else [torch.empty((T, N), dtype=torch.float32, device=x.device) for N in Ns]
    Wa = (ctypes.c_void_p * n)(*[W.data_ptr() for W in Ws])
    ya = (ctypes.c_void_p * n)(*[y.data_ptr() for y in ys])
    Na = (ctypes.c_int * n)(*Ns)
    check(lib().kata_gemv_q8_0_batch(n, Wa, ya, Na, _ptr(x), _xdtype(x), K, T, _stream(x)))
    return ys


# ----------------------------------------------------------------------------- prefill
def gemm_ptq1_f16(A: torch.Tensor, W: torch.Tensor, K: int, N: int, out_dtype=torch.float32,
                  out: torch.Tensor | None = None) -> torch.Tensor:
    if A.dtype != torch.float16:
        raise ValueError("A must be fp16")
    if A.dim() != 2 or A.shape[1] < K:
        raise ValueError(f"A must be [M][lda] with lda >= K={K}")
    M = A.shape[0]
    _need_bytes("W", W, _ptq1_bytes(K, N))
    if out is not None and (out.dim() != 2 or out.shape[0] < M or out.shape[1] < N):
        raise ValueError(f"out must be [>= {M}][>= {N}]")
    _need_gpu(A, W)
    C = out if out is not None else torch.empty((M, N), dtype=out_dtype, device=A.device)
    cdt = KATA_F16 if C.dtype == torch.float16 else KATA_F32
    check(lib().kata_gemm_ptq1_f16(_ptr(A), A.shape[1], _ptr(W), _ptr(C), cdt, C.shape[1], M, K, N, _stream(A)))
    return C


def gemm_q8_f16(A: torch.Tensor, W: torch.Tensor, K: int, N: int, out_dtype=torch.float32,
                out: torch.Tensor | None = None) -> torch.Tensor:
    """Exact fp16 GEMM over a Q8_0 matrix [N][K/32 * 34 B] (the MTP K/V catch-up)."""
    if A.dtype != torch.float16:
        raise ValueError("A must be fp16")
    if A.dim() != 2 or A.shape[1] < K:
        raise ValueError(f"A must be [M][lda] with lda >= K={K}")
    M = A.shape[0]
    _need_bytes("W", W, N * (K // Q8_GROUP) * Q8_BLOCK_BYTES)
    if out is not None and (out.dim() != 2 or out.shape[0] < M or out.shape[1] < N):
        raise ValueError(f"out must be [>= {M}][>= {N}]")
    _need_gpu(A, W)
    C = out if out is not None else torch.empty((M, N), dtype=out_dtype, device=A.device)
    cdt = KATA_F16 if C.dtype == torch.float16 else KATA_F32
    check(lib().kata_gemm_q8_0_f16(_ptr(A), A.shape[1], _ptr(W), _ptr(C), cdt, C.shape[1], M, K, N, _stream(A)))
    return C


def quant_rows(X: torch.Tensor, ldS: int | None = None, out=None):
    """int8 rows and group scales of X; `out` = (Q, SX) to write into existing tensors."""
    M, K = X.shape
    ldS = M if ldS is None else ldS
    if K % GROUP or ldS < M:
        raise ValueError(f"K={K} must be a multiple of {GROUP} and ldS={ldS} >= M={M}")
    if out is not None:
        _need_bytes("Q", out[0], M * K)
        _need_bytes("SX", out[1], (K // GROUP) * ldS * 4)
    _need_gpu(X)
    if out is not None:
        Q, SX = out
    else:
        Q = torch.empty((M, K), dtype=torch.int8, device=X.device)
        SX = torch.zeros((K // GROUP, ldS), dtype=torch.float32, device=X.device)
    check(lib().kata_quant_rows_i8(_ptr(X), _ptr(Q), _ptr(SX), M, K, ldS, _stream(X)))
    return Q, SX


def gemm_ptq1_i8(A8: torch.Tensor, SX: torch.Tensor, W: torch.Tensor, K: int, N: int,
                 out_dtype=torch.float32, out: torch.Tensor | None = None) -> torch.Tensor:
    M = A8.shape[0]
    if A8.dim() != 2 or A8.shape[1] != K:
        raise ValueError(f"A8 must be [M][K={K}]")
    if SX.dim() != 2 or SX.shape[0] < K // GROUP or SX.shape[1] < M:
        raise ValueError(f"SX must be [>= {K // GROUP}][ldS >= {M}]")
    _need_bytes("W", W, _ptq1_bytes(K, N))
    if out is not None and (out.dim() != 2 or out.shape[0] < M or out.shape[1] < N):
        raise ValueError(f"out must be [>= {M}][>= {N}]")
    _need_gpu(A8, SX, W)
    C = out if out is not None else torch.empty((M, N), dtype=out_dtype, device=A8.device)
    cdt = KATA_F16 if C.dtype == torch.float16 else KATA_F32
    check(lib().kata_gemm_ptq1_i8(_ptr(A8), _ptr(SX), SX.shape[1], _ptr(W), _ptr(C), cdt, C.shape[1],
                                  M, K, N, _stream(A8)))
    return C


def expand_f16(W: torch.Tensor, K: int, N: int) -> torch.Tensor:
    _need_bytes("W", W, _ptq1_bytes(K, N))
    _need_gpu(W)
    out = torch.empty((N, K), dtype=torch.float16, device=W.device)
    check(lib().kata_expand_ptq1_f16(_ptr(W), _ptr(out), K, N, _stream(W)))
    return out


def expand_i8(W: torch.Tensor, K: int, N: int):
    _need_bytes("W", W, _ptq1_bytes(K, N))
    _need_gpu(W)
    T8 = torch.empty((N, K), dtype=torch.int8, device=W.device)
    SW = torch.empty((N, K // GROUP), dtype=torch.float32, device=W.device)
    check(lib().kata_expand_ptq1_i8(_ptr(W), _ptr(T8), _ptr(SW), K, N, _stream(W)))
    return T8, SW


# ----------------------------------------------------------------------------- host packers
# ----------------------------------------------------------------------------- matmul input transform
def _fwht_out(out_dtype, half2: bool, M: int, W: int, device) -> torch.Tensor:
    """Output of an input transform: fp32/fp16 rows, half2 [W][2], or (uint8) the operand form."""
    if half2:
        return torch.empty((W, 2), dtype=torch.float16, device=device)
    if out_dtype == torch.uint8:
        n = gemv_xq_bytes(W, M)
        if n == 0:
            raise ValueError(f"W={W} M={M}: no operand form")
        return torch.empty(n, dtype=torch.uint8, device=device)
    return torch.empty((M, W), dtype=out_dtype, device=device)


def add_rms_fwht(x: torch.Tensor, gs: torch.Tensor, y: torch.Tensor | None = None, gamma: torch.Tensor | None = None,
                 out_dtype=torch.float32, half2: bool = False, want_xnew: bool = False, hout_dtype=torch.float32):
    """Residual add + RMSNorm + sign + 1024-block FWHT of fp32 rows x [M][W] (k_add_rms_fwht):
    returns (out, xnew or None, hout or None)."""
    _need_gpu(x, gs)
    M, W = x.shape
    out = _fwht_out(out_dtype, half2, M, W, x.device)
    xnew = torch.empty_like(x) if want_xnew else None
    hout = torch.empty((M, W), dtype=hout_dtype, device=x.device) if gamma is not None else None
    check(lib().kata_add_rms_fwht(_ptr(x), _ptr(y), _ptr(gs), _ptr(out), _xdtype(out),
                                  KATA_X_HALF2 if half2 else KATA_X_ROWS, _ptr(xnew), _ptr(gamma), _ptr(hout),
                                  KATA_F16 if hout_dtype == torch.float16 else KATA_F32, W, M, _stream(x)))
    return out, xnew, hout


def rms_fwht(src: torch.Tensor, gs: torch.Tensor, mode: int, src2: torch.Tensor | None = None,
             out_dtype=torch.float32, half2: bool = False):
    """The other input transforms (k_rms_fwht): mode 0 RMSNorm, 1 SwiGLU, 2 GDN head order, 3 plain."""
    _need_gpu(src, gs)
    M, W = src.shape
    out = _fwht_out(out_dtype, half2, M, W, src.device)
    check(lib().kata_rms_fwht(_ptr(src), _ptr(src2), _ptr(gs), _ptr(out), _xdtype(out),
                              KATA_X_HALF2 if half2 else KATA_X_ROWS, W, M, mode, _stream(src)))
    return out


def argmax(x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """Greedy argmax of fp32 logits (k_argmax): a device int32 tensor of one element."""
    _need_gpu(x)
    o = out if out is not None else torch.empty(1, dtype=torch.int32, device=x.device)
    check(lib().kata_argmax(_ptr(x), x.numel(), _ptr(o), _stream(x)))
    return o


def calib_empty(out: torch.Tensor, wgs: int = 0) -> None:
    """Empty kernel at the decode GEMV's launch geometry (the launch floor); out: int32 [>=1]."""
    _need_gpu(out)
    check(lib().kata_calib_empty(_ptr(out), wgs, _stream(out)))


def calib_read(buf: torch.Tensor, out: torch.Tensor, nbytes: int | None = None, wgs: int = 0) -> None:
    """Plain streaming read of nbytes (default: all) of buf at the decode GEMV's geometry."""
    _need_gpu(buf, out)
    n = _bytes(buf) if nbytes is None else nbytes
    _need_bytes("buf", buf, n)
    check(lib().kata_calib_read(_ptr(buf), n, _ptr(out), wgs, _stream(buf)))


def calib_read_cfg(buf: torch.Tensor, out: torch.Tensor, threads: int, wgs: int, inflight: int, nt: bool,
                   nbytes: int | None = None) -> None:
    """Plain streaming read at a given geometry (the sweep behind the read ceiling)."""
    _need_gpu(buf, out)
    n = _bytes(buf) if nbytes is None else nbytes
    _need_bytes("buf", buf, n)
    check(lib().kata_calib_read_cfg(_ptr(buf), n, _ptr(out), threads, wgs, inflight, int(nt), _stream(buf)))


def calib_read_peak(buf: torch.Tensor, out: torch.Tensor, nbytes: int | None = None) -> None:
    """Plain streaming read of nbytes (default: all) of buf at the fastest plain-read geometry."""
    _need_gpu(buf, out)
    n = _bytes(buf) if nbytes is None else nbytes
    _need_bytes("buf", buf, n)
    check(lib().kata_calib_read_peak(_ptr(buf), n, _ptr(out), _stream(buf)))


def calib_read_ptq1(W: torch.Tensor, K: int, N: int, out: torch.Tensor) -> None:
    """The decode GEMV's weight-load stream alone for the K x N PTQ1_0 matrix W at T = 1 (its
    loads in its order, nothing else): the rate its loop would reach if the rest were free."""
    _need_gpu(W, out)
    _need_bytes("W", W, N * (K // 128) * 28)
    check(lib().kata_calib_read_ptq1(_ptr(W), K, N, _ptr(out), _stream(W)))


def _np_ptr(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def quantize_ptq1(x: np.ndarray) -> np.ndarray:
    """Host quantize_row_ptq1_0_ref over the rows of a float32 [N][K] array."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    N, K = x.shape
    out = np.empty((N, K // GROUP * BLOCK_BYTES), np.uint8)
    check(lib().kata_quantize_ptq1_0(_np_ptr(x), _np_ptr(out), N, K))
    return out


def pack_ptq1(trits: np.ndarray, scales_f16: np.ndarray) -> np.ndarray:
    """Host packer: int8 trits [N][K] + fp16 scales [N][K/128] -> PTQ1_0 bytes."""
    trits = np.ascontiguousarray(trits, dtype=np.int8)
    N, K = trits.shape
    sc = np.ascontiguousarray(np.asarray(scales_f16, dtype=np.float16).view(np.uint16))
    out = np.empty((N, K // GROUP * BLOCK_BYTES), np.uint8)
    check(lib().kata_pack_ptq1_0(_np_ptr(trits), _np_ptr(sc), _np_ptr(out), N, K))
    return out
