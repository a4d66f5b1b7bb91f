"""GGUF v3 model files through the C ABI (kata_gguf_*): tensor index, metadata, and the
data region copied to device memory once, so matrices are byte offsets into it (the
reference's weight base + offset, src/engine.cpp:27-37)."""
from __future__ import annotations

import ctypes

import torch

from .capi import KataError, lib

GGML_F32, GGML_F16, GGML_Q8_0, GGML_PTQ1_0 = 0, 1, 8, 143


class GgufFile:
    def __init__(self, path: str):
        self._h = lib().kata_gguf_open(path.encode())
        if not self._h:
            raise KataError(lib().kata_last_error().decode())
        self.tensors = {}
        name, typ = ctypes.c_char_p(), ctypes.c_uint32()
        dims, off, nb = (ctypes.c_uint64 * 4)(), ctypes.c_uint64(), ctypes.c_uint64()
        for i in range(lib().kata_gguf_tensor_count(self._h)):
            if lib().kata_gguf_tensor(self._h, i, ctypes.byref(name), ctypes.byref(typ), dims, ctypes.byref(off),
                                      ctypes.byref(nb)):
                raise KataError(lib().kata_last_error().decode())
            self.tensors[name.value.decode()] = {"type": typ.value, "dims": list(dims), "offset": off.value,
                                                 "nbytes": nb.value}

    @property
    def data_bytes(self) -> int:
        return lib().kata_gguf_data_bytes(self._h)

    def get_int(self, key: str) -> int:
        v = ctypes.c_uint64()
        if lib().kata_gguf_get_int(self._h, key.encode(), ctypes.byref(v)):
            raise KeyError(key)
        return v.value

    def get_str(self, key: str) -> str | None:
        s = lib().kata_gguf_get_str(self._h, key.encode())
        return None if s is None else s.decode()

    def upload(self, device) -> torch.Tensor:
        """The data region as one device uint8 tensor (matrices at their `offset`)."""
        buf = torch.empty(max(1, self.data_bytes), dtype=torch.uint8, device=device)
        if lib().kata_gguf_upload_into(self._h, ctypes.c_void_p(buf.data_ptr()), buf.numel()):
            raise KataError(lib().kata_last_error().decode())
        return buf

    def close(self):
        if self._h:
            lib().kata_gguf_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
