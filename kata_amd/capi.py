"""ctypes binding of libkata_amd.so (the C ABI declared in include/kata_amd.h).

The library is loaded from this package directory only; if it is missing the import of
any op raises — there is no CPU fallback on the product path.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "libkata_amd.so")
_lib = None

KATA_F32, KATA_F16, KATA_XQ = 0, 1, 2   # KATA_XQ: the decode GEMV's operand form
KATA_X_ROWS, KATA_X_HALF2 = 0, 1
KATA_EINVAL, KATA_ELAUNCH = -1, -2
KATA_FORM_DECODE, KATA_FORM_PREFILL, KATA_FORM_VERIFY = 0, 1, 2


class KataError(RuntimeError):
    def __init__(self, rc: int, msg: str):
        super().__init__(f"kata_amd error {rc}: {msg}")
        self.rc = rc


def library_path() -> str:
    return _SO


P, I, I64, U64, U32, SZ = (ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_uint64,
                           ctypes.c_uint32, ctypes.c_size_t)

# every symbol of include/kata_amd.h with its ctypes signature
SIGNATURES = {
    "kata_last_error": (ctypes.c_char_p, []),
    "kata_version": (ctypes.c_char_p, []),
    "kata_gemv_ptq1": (I, [P, P, I, I, P, I, I, I, P]),
    "kata_gemv_ptq1_max_k": (I, [I]),
    "kata_gemv_ptq1_batch": (I, [I, P, P, P, P, I, I, I, I, P]),
    "kata_gemv_q8_0": (I, [P, P, I, P, I, I, I, P]),
    "kata_gemv_q8_0_batch": (I, [I, P, P, P, P, I, I, I, P]),
    "kata_dispatch_gemv_q8": (I, [P, I, P, P, I, P, P, I, I, P]),
    "kata_gemm_ptq1_f16": (I, [P, I, P, P, I, I, I, I, I, P]),
    "kata_gemm_q8_0_f16": (I, [P, I, P, P, I, I, I, I, I, P]),
    "kata_quant_rows_i8": (I, [P, P, P, I, I, I, P]),
    "kata_gemm_ptq1_i8": (I, [P, P, I, P, P, I, I, I, I, I, P]),
    "kata_expand_ptq1_f16": (I, [P, P, I, I, P]),
    "kata_expand_ptq1_i8": (I, [P, P, P, I, I, P]),
    "kata_add_rms_fwht": (I, [P, P, P, P, I, I, P, P, P, I, I, I, P]),
    "kata_rms_fwht": (I, [P, P, P, P, I, I, I, I, I, P]),
    "kata_argmax": (I, [P, I, P, P]),
    "kata_release_stream": (I, [P]),
    "kata_quantize_ptq1_0": (I, [P, P, I64, I64]),
    "kata_pack_ptq1_0": (I, [P, P, P, I64, I64]),
    "kata_gguf_open": (P, [ctypes.c_char_p]),
    "kata_gguf_close": (None, [P]),
    "kata_gguf_tensor_count": (I64, [P]),
    "kata_gguf_data_bytes": (U64, [P]),
    "kata_gguf_tensor": (I, [P, I64, P, P, P, P, P]),
    "kata_gguf_find": (I64, [P, ctypes.c_char_p]),
    "kata_gguf_get_int": (I, [P, ctypes.c_char_p, P]),
    "kata_gguf_get_str": (ctypes.c_char_p, [P, ctypes.c_char_p]),
    "kata_gguf_upload": (I, [P, P]),
    "kata_gguf_upload_into": (I, [P, P, U64]),
    "kata_gguf_free_device": (I, [P]),
    "kata_gemv_ptq1_wide": (I, [P, P, I, P, I, I, I, P]),
    "kata_gemv_ptq1_wide_noalloc": (I, [P, P, I, P, I, I, I, P]),
    "kata_gemv_ptq1_wide_batch": (I, [I, P, P, P, P, I, I, I, P]),
    "kata_gemv_ptq1_wide_noalloc_scratch_bytes": (SZ, []),
    "kata_dispatch_create": (P, [P]),
    "kata_dispatch_destroy": (None, [P]),
    "kata_dispatch_set_i8": (I, [P, ctypes.c_char_p]),
    "kata_dispatch_i8": (I, [P, ctypes.c_char_p]),
    "kata_dispatch_i8_mask": (U32, [P]),
    "kata_dispatch_gemv": (I, [P, U64, P, P, I, I, P]),
    "kata_dispatch_prefill": (I, [P, U64, P, P, I, I, I, ctypes.c_char_p, P, P, I, P]),
    "kata_dispatch_ffn_decode": (I, [P, U64, U64, U64, P, P, P, P, P, P, P, I, I, P]),
    "kata_dispatch_ffn_prefill": (I, [P, U64, U64, U64, P, P, P, P, P, P, P, I, I, I, P]),
    "kata_ffn_prefill_work_bytes": (SZ, [I, I, I]),
    "kata_dispatch_ffn_verify": (I, [P, U64, U64, U64, P, P, P, P, P, P, P, I, I, I, P]),
    "kata_ffn_verify_work_bytes": (SZ, [I, I, I]),
    "kata_dispatch_in": (I, [P, I, I, P, P, P, P, P, P, P, P, P, P, I, P, I, I, P]),
    "kata_dispatch_out": (I, [P, I, U64, ctypes.c_char_p, P, P, I, P, P, P, I, I, I, P]),
    "kata_dispatch_work_bytes": (SZ, [I, I, I]),
    "kata_calib_empty": (I, [P, I, P]),
    "kata_calib_read": (I, [P, SZ, P, I, P]),
    "kata_calib_read_peak": (I, [P, SZ, P, P]),
    "kata_calib_read_cfg": (I, [P, SZ, P, I, I, I, I, P]),
    "kata_calib_read_ptq1": (I, [P, I, I, P, P]),
    "kata_gemv_xq_bytes": (SZ, [I, I]),
    "kata_gemv_prepare_x": (I, [P, I, I, I, I, P, P]),
}


def lib():
    """Loads libkata_amd.so (raises if it was not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(_SO):
            raise ImportError(f"{_SO} is missing: run `python -m kata_amd.build` (no CPU fallback exists)")
        L = ctypes.CDLL(_SO)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype, f.argtypes = res, args
        _lib = L
    return _lib


def check(rc: int) -> None:
    if rc != 0:
        raise KataError(rc, lib().kata_last_error().decode())
