"""Engine-side matmul dispatch over the C ABI, mirroring the reference engine's helpers.

`Dispatch` binds one device weight buffer (the reference binds the whole mmapped GGUF,
src/engine.cpp:27) and maps (byte offset, K, N, matrix name) to the kernels:
  gemv(wOff, x, y, K, N)            <- Engine::dGemvPtq1 (src/engine.cpp:97-101)
  prefill(wOff, A, C, K, N, name)   <- Engine::dExpandGemm (src/engine.cpp:208-219)
  set_i8(spec) / i8(name)           <- Engine::setI8 / i8 (src/engine.cpp:529-537,
                                       src/engine.h:89-95)
  ffn_decode / ffn_prefill / ffn_verify  <- the FFN block of Engine::step, prefill and
                                       verifyWide (src/engine.cpp:176-182, 247-300, 627-629)
Errors raise KataError instead of the reference's exit(1).
"""
from __future__ import annotations

import ctypes

import torch

from .capi import KataError, check, lib
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


def ffn_prefill_work_bytes(H: int, F: int, M: int) -> int:
    return int(lib().kata_ffn_prefill_work_bytes(H, F, M))
