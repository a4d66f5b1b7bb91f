"""Engine-side matmul dispatch over the C ABI, mirroring the reference engine's helpers.

`Dispatch` binds one device weight buffer (the reference binds the whole mmapped GGUF,
src/engine.cpp:27) and maps (byte offset, K, N, matrix name) to the kernels:
  gemv(wOff, x, y, K, N)            <- Engine::dGemvPtq1 (src/engine.cpp:97-101)
  prefill(wOff, A, C, K, N, name)   <- Engine::dExpandGemm (src/engine.cpp:208-219)
  set_i8(spec) / i8(name)           <- Engine::setI8 / i8 (src/engine.cpp:529-537,
                                       src/engine.h:89-95)
  ffn_decode / ffn_prefill / ffn_verify  <- the FFN block of Engine::step, prefill and
                                       verifyWide (src/engine.cpp:176-182, 247-300, 627-629)
  sub_in / sub_out                  <- the matmul halves of any sublayer (GDN: qkv + z and
                                       ssm_out; GQA: q + k + v and o; FFN: gate + up and
                                       down) in the decode, prefill and verify forms
                                       (src/engine.cpp:150-182, 247-300, 454-491)
Errors raise KataError instead of the reference's exit(1).
"""
from __future__ import annotations

import ctypes

import torch

from .capi import KATA_FORM_DECODE, KATA_FORM_PREFILL, KATA_FORM_VERIFY, KataError, check, lib
from .ops import _ptr, _stream

I8_NAMES = ("qkv", "z", "ssmout", "wq", "wk", "wv", "wo", "gate", "up", "down")


class Dispatch:
    def __init__(self, wbuf: torch.Tensor):
        if not wbuf.is_cuda or wbuf.dtype != torch.uint8:
            raise ValueError("weight buffer must be a uint8 device tensor")
        self.wbuf = wbuf
        h = lib().kata_dispatch_create(_ptr(wbuf))
        if not h:
            raise KataError(-1, lib().kata_last_error().decode())
        self._h = ctypes.c_void_p(h)

    def close(self):
        if self._h:
            lib().kata_dispatch_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- int8 selection
    def set_i8(self, spec: str) -> None:
        check(lib().kata_dispatch_set_i8(self._h, spec.encode()))

    def i8(self, name: str) -> bool:
        return bool(lib().kata_dispatch_i8(self._h, name.encode()))

    @property
    def i8_mask(self) -> int:
        return int(lib().kata_dispatch_i8_mask(self._h))

    # ---- matmuls
    def gemv(self, wOff: int, x: torch.Tensor, y: torch.Tensor, K: int, N: int) -> None:
        check(lib().kata_dispatch_gemv(self._h, wOff, _ptr(x), _ptr(y), K, N, _stream(self.wbuf)))

    def gemv_q8(self, offs, x: torch.Tensor, outs, K: int, Ns) -> None:
        """The MTP block's `gq` (src/engine.cpp:351) for 1..4 Q8_0 matrices reading x [T][K]."""
        n = len(offs)
        T = x.shape[0]
        oa = (ctypes.c_uint64 * n)(*offs)
        ya = (ctypes.c_void_p * n)(*[o.data_ptr() for o in outs])
        Na = (ctypes.c_int * n)(*Ns)
        check(lib().kata_dispatch_gemv_q8(self._h, n, oa, _ptr(x), 1 if x.dtype == torch.float16 else 0, ya, Na, K, T,
                                          _stream(self.wbuf)))

    def prefill(self, wOff: int, A: torch.Tensor, C: torch.Tensor, K: int, N: int, name: str,
                A8: torch.Tensor | None = None, SX: torch.Tensor | None = None) -> None:
        M = A.shape[0]
        ldS = SX.shape[1] if SX is not None else M
        check(lib().kata_dispatch_prefill(self._h, wOff, _ptr(A), _ptr(C), M, K, N, name.encode(),
                                          _ptr(A8), _ptr(SX), ldS, _stream(self.wbuf)))

    # ---- layer level: the FFN sublayer (src/engine.cpp:176-182 decode, :247-300 prefill)
    def ffn_decode(self, offGate: int, offUp: int, offDown: int, x: torch.Tensor, y: torch.Tensor | None,
                   gs_in: torch.Tensor, gs_down: torch.Tensor, H: int, F: int, out: torch.Tensor | None = None,
                   xnew: torch.Tensor | None = None, work: torch.Tensor | None = None) -> torch.Tensor:
        """out = W_down H(silu(W_gate h) * (W_up h) * gs_down), h = H(rmsnorm(x + y) * gs_in)."""
        dev = x.device
        if out is None:
            out = torch.empty(H, dtype=torch.float32, device=dev)
        if work is None:
            work = torch.empty(H + 3 * F, dtype=torch.float32, device=dev)
        check(lib().kata_dispatch_ffn_decode(self._h, offGate, offUp, offDown, _ptr(x), _ptr(y), _ptr(xnew),
                                             _ptr(gs_in), _ptr(gs_down), _ptr(work), _ptr(out), H, F,
                                             _stream(self.wbuf)))
        return out

    def ffn_prefill(self, offGate: int, offUp: int, offDown: int, x: torch.Tensor, y: torch.Tensor | None,
                    gs_in: torch.Tensor, gs_down: torch.Tensor, H: int, F: int, out: torch.Tensor | None = None,
                    xnew: torch.Tensor | None = None, work: torch.Tensor | None = None) -> torch.Tensor:
        """The FFN sublayer over M = x.shape[0] rows; GEMMs on the paths set_i8 selected."""
        M = x.shape[0]
        dev = x.device
        if out is None:
            out = torch.empty((M, H), dtype=torch.float32, device=dev)
        if work is None:
            work = torch.empty(ffn_prefill_work_bytes(H, F, M), dtype=torch.uint8, device=dev)
        check(lib().kata_dispatch_ffn_prefill(self._h, offGate, offUp, offDown, _ptr(x), _ptr(y), _ptr(xnew),
                                              _ptr(gs_in), _ptr(gs_down), _ptr(work), _ptr(out), H, F, M,
                                              _stream(self.wbuf)))
        return out

    def ffn_verify(self, offGate: int, offUp: int, offDown: int, x: torch.Tensor, y: torch.Tensor | None,
                   gs_in: torch.Tensor, gs_down: torch.Tensor, H: int, F: int, out: torch.Tensor | None = None,
                   xnew: torch.Tensor | None = None, work: torch.Tensor | None = None) -> torch.Tensor:
        """The FFN sublayer for T = x.shape[0] <= 8 verification tokens (wide GEMVs)."""
        T = x.shape[0]
        dev = x.device
        if out is None:
            out = torch.empty((T, H), dtype=torch.float32, device=dev)
        if work is None:
            work = torch.empty(int(lib().kata_ffn_verify_work_bytes(H, F, T)), dtype=torch.uint8, device=dev)
        check(lib().kata_dispatch_ffn_verify(self._h, offGate, offUp, offDown, _ptr(x), _ptr(y), _ptr(xnew),
                                             _ptr(gs_in), _ptr(gs_down), _ptr(work), _ptr(out), H, F, T,
                                             _stream(self.wbuf)))
        return out


    # ---- layer level: any sublayer's matmul halves
    _FORMS = {"decode": KATA_FORM_DECODE, "prefill": KATA_FORM_PREFILL, "verify": KATA_FORM_VERIFY}

    def sub_in(self, form: str, mats, x: torch.Tensor, y: torch.Tensor | None, gs: torch.Tensor,
               xnew: torch.Tensor | None = None, gamma: torch.Tensor | None = None,
               hout: torch.Tensor | None = None, work: torch.Tensor | None = None):
        """h = H(rmsnorm(x + y) * gs) over M = x.shape[0] rows (decode: M == 1), then W_i h for
        mats = [(offset, N, name)]: returns the fp32 outputs [M][N_i]."""
        M, H = x.shape
        dev = x.device
        n = len(mats)
        outs = [torch.empty((M, N), dtype=torch.float32, device=dev) for _, N, _ in mats]
        if work is None:
            work = torch.empty(dispatch_work_bytes(form, H, M), dtype=torch.uint8, device=dev)
        offs = (ctypes.c_uint64 * n)(*[o for o, _, _ in mats])
        Ns = (ctypes.c_int * n)(*[N for _, N, _ in mats])
        names = (ctypes.c_char_p * n)(*[nm.encode() for _, _, nm in mats])
        optr = (ctypes.c_void_p * n)(*[o.data_ptr() for o in outs])
        hdt = 1 if hout is not None and hout.dtype == torch.float16 else 0
        check(lib().kata_dispatch_in(self._h, self._FORMS[form], n, offs, Ns, names, optr, _ptr(x), _ptr(y), _ptr(xnew),
                                     _ptr(gs), _ptr(gamma), _ptr(hout), hdt, _ptr(work), H, M, _stream(self.wbuf)))
        return outs

    def sub_out(self, form: str, off: int, name: str, src: torch.Tensor, src2: torch.Tensor | None, mode: int,
                gs: torch.Tensor, H: int, work: torch.Tensor | None = None) -> torch.Tensor:
        """t = H(transform_mode(src, src2) * gs), then W t: fp32 [M][H]."""
        M, W = src.shape
        dev = src.device
        out = torch.empty((M, H), dtype=torch.float32, device=dev)
        if work is None:
            work = torch.empty(dispatch_work_bytes(form, W, M), dtype=torch.uint8, device=dev)
        check(lib().kata_dispatch_out(self._h, self._FORMS[form], off, name.encode(), _ptr(src), _ptr(src2), mode,
                                      _ptr(gs), _ptr(work), _ptr(out), W, H, M, _stream(self.wbuf)))
        return out


def dispatch_work_bytes(form: str, K: int, M: int) -> int:
    return int(lib().kata_dispatch_work_bytes(Dispatch._FORMS[form], K, M))


def ffn_prefill_work_bytes(H: int, F: int, M: int) -> int:
    return int(lib().kata_ffn_prefill_work_bytes(H, F, M))
