"""CPU-side checks of the C ABI: the library loads, exports every symbol the header
declares, validates arguments before touching the GPU, and its host packers and the
int8 selection logic match the reference's behaviour.  No kernel is launched here."""
import ctypes
import os
import re

import numpy as np
import pytest

from kata_amd import capi as L
from kata_amd.capi import KATA_EINVAL
from oracle import oracle as orc

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_symbols():
    txt = open(os.path.join(ROOT, "include", "kata_amd.h")).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(kata_[a-z0-9_]+)\s*\(", txt)))


def test_library_exports_every_header_symbol():
    syms = header_symbols()
    assert len(syms) >= 19
    lib = L.lib()
    for s in syms:
        assert hasattr(lib, s), s
        assert s in L.SIGNATURES, f"{s} has no ctypes signature"
    assert set(L.SIGNATURES) == set(syms)


def test_exports_with_nm():
    import subprocess
    out = subprocess.run(["nm", "-D", "--defined-only", L.library_path()], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\bT (kata_[a-z0-9_]+)\b", out))
    assert set(header_symbols()) <= exported


def test_version():
    assert b"gfx950" in L.lib().kata_version()


FAKE = ctypes.c_void_p(0x10000)   # never dereferenced: validation fails first


@pytest.mark.parametrize("K,N,T,dt,layout", [
    (100, 8, 1, 0, 0),     # K not a multiple of 128
    (0, 8, 1, 0, 0),
    (128, 0, 1, 0, 0),     # N = 0
    (128, 8, 3, 0, 0),     # T = 3
    (128, 8, 1, 5, 0),     # bad dtype
    (128, 8, 1, 1, 1),     # half2 needs T = 2
    (128, 8, 2, 0, 1),     # half2 needs fp16
    (-1, 8, 1, 0, 0),      # K one group beyond the LDS-resident activation limit (T=1)
    (-2, 8, 2, 1, 0),      # same for T=2
])
def test_gemv_rejects_bad_arguments(K, N, T, dt, layout):
    if K < 0:
        K = L.lib().kata_gemv_ptq1_max_k(-K) + 128
    rc = L.lib().kata_gemv_ptq1(FAKE, FAKE, dt, layout, FAKE, K, N, T, None)
    assert rc == KATA_EINVAL
    assert L.lib().kata_last_error()


def test_other_entry_points_reject_bad_shapes():
    lib = L.lib()
    assert lib.kata_gemv_ptq1(None, FAKE, 0, 0, FAKE, 128, 8, 1, None) == KATA_EINVAL
    assert lib.kata_gemv_q8_0(FAKE, FAKE, 0, FAKE, 48, 8, 1, None) == KATA_EINVAL
    Wa = (ctypes.c_void_p * 5)(*([0x10000] * 5))
    Na = (ctypes.c_int * 5)(*([8] * 5))
    for count in (0, 5):                                   # 1..4 matrices per launch
        assert lib.kata_gemv_ptq1_batch(count, Wa, Wa, Na, FAKE, 0, 0, 128, 1, None) == KATA_EINVAL
    Na[1] = 0                                              # every N must be positive
    assert lib.kata_gemv_ptq1_batch(2, Wa, Wa, Na, FAKE, 0, 0, 128, 1, None) == KATA_EINVAL
    assert lib.kata_gemm_ptq1_f16(FAKE, 120, FAKE, FAKE, 0, 8, 4, 128, 8, None) == KATA_EINVAL   # lda < K
    assert lib.kata_gemm_ptq1_f16(FAKE, 128, FAKE, FAKE, 0, 4, 4, 128, 8, None) == KATA_EINVAL   # ldc < N
    assert lib.kata_gemm_ptq1_f16(FAKE, 136, FAKE, FAKE, 0, 8, 4, 136, 8, None) == KATA_EINVAL   # K % 128
    assert lib.kata_quant_rows_i8(FAKE, FAKE, FAKE, 4, 128, 2, None) == KATA_EINVAL            # ldS < M
    assert lib.kata_gemm_ptq1_i8(FAKE, FAKE, 4, FAKE, FAKE, 0, 4, 4, 128, 8, None) == KATA_EINVAL  # ldc < N
    assert lib.kata_gemv_ptq1(FAKE, ctypes.c_void_p(0x10008), 1, 0, FAKE, 128, 8, 1, None) == KATA_EINVAL  # x align
    # matmul input transform: W % 1024, half2 only for fp16 with M == 2, mode 2 only at W = 6144,
    # gamma and hout together
    assert lib.kata_add_rms_fwht(FAKE, None, FAKE, FAKE, 0, 0, None, None, None, 0, 1000, 1, None) == KATA_EINVAL
    assert lib.kata_add_rms_fwht(FAKE, None, FAKE, FAKE, 0, 1, None, None, None, 0, 1024, 2, None) == KATA_EINVAL
    assert lib.kata_add_rms_fwht(FAKE, None, FAKE, FAKE, 1, 1, None, None, None, 0, 1024, 3, None) == KATA_EINVAL
    assert lib.kata_add_rms_fwht(FAKE, None, FAKE, FAKE, 0, 0, None, FAKE, None, 0, 1024, 1, None) == KATA_EINVAL
    assert lib.kata_rms_fwht(FAKE, None, FAKE, FAKE, 0, 0, 5120, 1, 2, None) == KATA_EINVAL
    assert lib.kata_rms_fwht(FAKE, None, FAKE, FAKE, 0, 0, 5120, 1, 1, None) == KATA_EINVAL   # mode 1 needs src2
    assert lib.kata_rms_fwht(FAKE, None, FAKE, FAKE, 0, 0, 5120, 1, 4, None) == KATA_EINVAL
    assert lib.kata_calib_read_ptq1(FAKE, 5000, 64, FAKE, None) == KATA_EINVAL        # K % 128
    assert lib.kata_calib_read_ptq1(FAKE, 5120, 0, FAKE, None) == KATA_EINVAL
    assert lib.kata_calib_read_ptq1(FAKE, 5120, 2_000_000, FAKE, None) == KATA_EINVAL  # >= 2^31 bytes
    assert lib.kata_calib_read_ptq1(ctypes.c_void_p(0x10008), 5120, 64, FAKE, None) == KATA_EINVAL  # alignment
    # the 27B shapes (K up to 17408) must fit for both T
    assert lib.kata_gemv_ptq1_max_k(1) >= 17408 and lib.kata_gemv_ptq1_max_k(2) >= 17408
    assert lib.kata_gemv_ptq1_max_k(1) % 128 == 0 and lib.kata_gemv_ptq1_max_k(2) % 128 == 0
    assert lib.kata_gemv_ptq1_max_k(3) == 0


def test_host_pack_matches_oracle_and_golden(golden):
    from kata_amd import ops
    W = ops.pack_ptq1(golden["ptq1_trits"], golden["ptq1_scales"])
    assert np.array_equal(W, golden["ptq1_W"])
    rng = np.random.default_rng(5)
    t = rng.integers(-1, 2, (33, 640)).astype(np.int8)
    s = np.abs(rng.normal(0, 0.02, (33, 5))).astype(np.float16)
    assert np.array_equal(ops.pack_ptq1(t, s), orc.pack(t, s))


def test_host_pack_rejects_non_trits():
    from kata_amd import ops
    from kata_amd.capi import KataError
    t = np.zeros((1, 128), np.int8); t[0, 3] = 2
    with pytest.raises(KataError):
        ops.pack_ptq1(t, np.ones((1, 1), np.float16))


def test_host_quantize_matches_oracle():
    from kata_amd import ops
    rng = np.random.default_rng(6)
    X = rng.standard_normal((9, 384)).astype(np.float32)
    X[2, :128] = 0.0                      # amax = 0 block
    X[3, 5] = 0.5 * np.abs(X[3, :128]).max()   # a rounding threshold value
    assert np.array_equal(ops.quantize_ptq1(X), orc.quantize(X))


def test_dispatch_i8_selection():
    lib = L.lib()
    h = ctypes.c_void_p(lib.kata_dispatch_create(FAKE))
    try:
        names = ["qkv", "z", "ssmout", "wq", "wk", "wv", "wo", "gate", "up", "down"]
        assert lib.kata_dispatch_set_i8(h, b"ffn") == 0
        assert [n for n in names if lib.kata_dispatch_i8(h, n.encode())] == ["gate", "up"]
        assert lib.kata_dispatch_set_i8(h, b"all") == 0
        assert lib.kata_dispatch_i8_mask(h) == (1 << 10) - 1
        assert lib.kata_dispatch_set_i8(h, b"down,wq") == 0
        assert lib.kata_dispatch_i8_mask(h) == (1 << 9) | (1 << 3)
        assert lib.kata_dispatch_set_i8(h, b"none") == 0 and lib.kata_dispatch_i8_mask(h) == 0
        assert lib.kata_dispatch_set_i8(h, b"") == 0 and lib.kata_dispatch_i8_mask(h) == 0
        assert lib.kata_dispatch_set_i8(h, b"gate,bogus") == KATA_EINVAL
        assert lib.kata_dispatch_set_i8(h, b"gate,,up") == KATA_EINVAL
        assert not lib.kata_dispatch_i8(h, b"lm_head")
    finally:
        lib.kata_dispatch_destroy(h)


def test_dispatch_ffn_rejects():
    """The FFN sublayer entry points validate before any launch (no GPU needed)."""
    lib = L.lib()
    h = ctypes.c_void_p(lib.kata_dispatch_create(FAKE))
    try:
        p = FAKE
        assert lib.kata_dispatch_ffn_decode(h, 0, 0, 0, p, None, None, p, p, p, p, 2048, 3000, None) == KATA_EINVAL
        assert lib.kata_dispatch_ffn_decode(h, 0, 0, 0, None, None, None, p, p, p, p, 2048, 3072, None) == KATA_EINVAL
        assert lib.kata_dispatch_ffn_decode(None, 0, 0, 0, p, None, None, p, p, p, p, 2048, 3072, None) == KATA_EINVAL
        assert lib.kata_dispatch_ffn_prefill(h, 0, 0, 0, p, None, None, p, p, p, p, 2048, 3072, 0, None) == KATA_EINVAL
        assert lib.kata_dispatch_ffn_prefill(h, 0, 0, 0, p, None, None, p, None, p, p, 2048, 3072, 4, None) == KATA_EINVAL
        assert lib.kata_dispatch_ffn_verify(h, 0, 0, 0, p, None, None, p, p, p, p, 2048, 3072, 9, None) == KATA_EINVAL
        assert lib.kata_dispatch_ffn_verify(h, 0, 0, 0, p, None, None, p, p, p, p, 2000, 3072, 2, None) == KATA_EINVAL
    finally:
        lib.kata_dispatch_destroy(h)
    # h and t in the wide GEMV's operand form (2080 B per 128-block), g and u fp32
    assert lib.kata_ffn_verify_work_bytes(1024, 2048, 3) == 8 * 2080 + 3 * 2048 * 8 + 16 * 2080
    # g, u fp32 + h, t fp16 + int8 rows + 16 alignment + scales
    assert lib.kata_ffn_prefill_work_bytes(1024, 2048, 8) == 8 * 2048 * 8 + 8 * 1024 * 2 + 8 * 2048 * 2 + 8 * 2048 + 16 + 16 * 8 * 4


def test_dispatch_sub_rejects():
    """The sublayer halves validate form, row count, widths and names before any launch."""
    lib = L.lib()
    h = ctypes.c_void_p(lib.kata_dispatch_create(FAKE))
    p = FAKE
    offs = (ctypes.c_uint64 * 2)(0, 100)
    Ns = (ctypes.c_int * 2)(1024, 1024)
    outs = (ctypes.c_void_p * 2)(0x10000, 0x20000)

    def sub_in(form, names, H=2048, M=1, count=2):
        nm = (ctypes.c_char_p * 2)(*[n.encode() for n in names])
        return lib.kata_dispatch_in(h, form, count, offs, Ns, nm, outs, p, None, None, p, None, None, 0, p, H, M, None)
    try:
        assert sub_in(3, ["wq", "wk"]) == KATA_EINVAL                  # unknown form
        assert sub_in(0, ["wq", "wk"], M=2) == KATA_EINVAL             # decode is one row
        assert sub_in(2, ["wq", "wk"], M=9) == KATA_EINVAL             # verify holds <= 8 tokens
        assert sub_in(1, ["wq", "wk"], M=0) == KATA_EINVAL
        assert sub_in(1, ["wq", "wk"], H=2000, M=4) == KATA_EINVAL     # H a multiple of 1024
        assert sub_in(1, ["wq", "lm_head"], M=4) == KATA_EINVAL        # names from the i8 set
        assert sub_in(1, ["wq", "wk"], M=4, count=5) == KATA_EINVAL
        out = lib.kata_dispatch_out
        assert out(h, 0, 0, b"wo", p, None, 4, p, p, p, 6144, 5120, 1, None) == KATA_EINVAL     # mode 1..3
        assert out(h, 0, 0, b"bogus", p, None, 3, p, p, p, 6144, 5120, 1, None) == KATA_EINVAL
        assert out(h, 2, 0, b"wo", p, None, 3, p, p, p, 6144, 5120, 9, None) == KATA_EINVAL
        assert out(h, 1, 0, b"wo", p, None, 3, p, p, p, 6000, 5120, 4, None) == KATA_EINVAL
        assert out(h, 1, 0, b"wo", p, None, 3, p, p, p, 6144, 0, 4, None) == KATA_EINVAL
        assert out(h, 1, 0, b"wo", None, None, 3, p, p, p, 6144, 5120, 4, None) == KATA_EINVAL
    finally:
        lib.kata_dispatch_destroy(h)
    assert lib.kata_dispatch_work_bytes(0, 5120, 1) == 4 * 5120
    assert lib.kata_dispatch_work_bytes(2, 5120, 3) == 40 * 2080          # the wide operand form
    assert lib.kata_dispatch_work_bytes(2, 5120, 1) == 10560               # the decode operand form (T = 1)
    assert lib.kata_dispatch_work_bytes(1, 5120, 5) == 2 * 5 * 5120 + 5 * 5120 + 4 * 40 * 5
    assert lib.kata_dispatch_work_bytes(3, 5120, 5) == 0


def test_gemv_wide_rejects():
    lib = L.lib()
    p = FAKE
    assert lib.kata_gemv_ptq1_wide(p, p, 1, p, 1024, 16, 0, None) == KATA_EINVAL
    assert lib.kata_gemv_ptq1_wide(p, p, 1, p, 1024, 16, 9, None) == KATA_EINVAL
    assert lib.kata_gemv_ptq1_wide(p, p, 1, p, 1000, 16, 4, None) == KATA_EINVAL
    assert lib.kata_gemv_ptq1_wide(p, p, 1, p, 1024, 0, 4, None) == KATA_EINVAL
    assert lib.kata_gemv_ptq1_wide(p, p, 7, p, 1024, 16, 4, None) == KATA_EINVAL
    assert lib.kata_gemv_ptq1_wide(p, ctypes.c_void_p(0x10008), 1, p, 1024, 16, 4, None) == KATA_EINVAL
    assert lib.kata_gemv_ptq1_wide(None, p, 1, p, 1024, 16, 4, None) == KATA_EINVAL


def test_gemv_wide_batch_rejects():
    lib = L.lib()
    p = FAKE

    def arr(ctype, vals):
        return (ctype * len(vals))(*vals)

    W2 = arr(ctypes.c_void_p, [FAKE.value, FAKE.value])
    y2 = arr(ctypes.c_void_p, [FAKE.value, FAKE.value])
    N2 = arr(ctypes.c_int, [16, 32])
    call = lib.kata_gemv_ptq1_wide_batch
    assert call(0, W2, y2, N2, p, 1, 1024, 4, None) == KATA_EINVAL            # count
    assert call(5, W2, y2, N2, p, 1, 1024, 4, None) == KATA_EINVAL
    assert call(2, W2, y2, N2, p, 1, 1024, 9, None) == KATA_EINVAL            # T
    assert call(2, W2, y2, N2, p, 1, 1000, 4, None) == KATA_EINVAL            # K % 128
    assert call(2, W2, y2, N2, p, 7, 1024, 4, None) == KATA_EINVAL            # x dtype
    assert call(2, W2, y2, N2, ctypes.c_void_p(0x10008), 1, 1024, 4, None) == KATA_EINVAL
    assert call(2, None, y2, N2, p, 1, 1024, 4, None) == KATA_EINVAL
    assert call(2, W2, y2, arr(ctypes.c_int, [16, 0]), p, 1, 1024, 4, None) == KATA_EINVAL
    assert call(2, arr(ctypes.c_void_p, [FAKE.value, 0x10002]), y2, N2, p, 1, 1024, 4, None) == KATA_EINVAL
    assert call(2, W2, arr(ctypes.c_void_p, [FAKE.value, None]), N2, p, 1, 1024, 4, None) == KATA_EINVAL


def test_gemv_q8_batch_rejects():
    lib = L.lib()
    p = FAKE

    def arr(ctype, vals):
        return (ctype * len(vals))(*vals)

    W2 = arr(ctypes.c_void_p, [FAKE.value, FAKE.value])
    y2 = arr(ctypes.c_void_p, [FAKE.value, FAKE.value])
    N2 = arr(ctypes.c_int, [16, 32])
    call = lib.kata_gemv_q8_0_batch
    assert call(0, W2, y2, N2, p, 1, 1024, 1, None) == KATA_EINVAL            # count
    assert call(5, W2, y2, N2, p, 1, 1024, 1, None) == KATA_EINVAL
    assert call(2, W2, y2, N2, p, 1, 1024, 3, None) == KATA_EINVAL            # T
    assert call(2, W2, y2, N2, p, 1, 1000, 1, None) == KATA_EINVAL            # K % 32
    assert call(2, W2, y2, N2, p, 7, 1024, 1, None) == KATA_EINVAL            # x dtype
    assert call(2, W2, y2, N2, ctypes.c_void_p(0x10008), 1, 1024, 1, None) == KATA_EINVAL
    assert call(2, None, y2, N2, p, 1, 1024, 1, None) == KATA_EINVAL
    assert call(2, W2, y2, arr(ctypes.c_int, [16, 0]), p, 1, 1024, 1, None) == KATA_EINVAL
    assert call(2, arr(ctypes.c_void_p, [FAKE.value, 0x10001]), y2, N2, p, 1, 1024, 1, None) == KATA_EINVAL
    assert call(2, W2, arr(ctypes.c_void_p, [FAKE.value, None]), N2, p, 1, 1024, 1, None) == KATA_EINVAL
    assert lib.kata_dispatch_gemv_q8(None, 1, arr(ctypes.c_uint64, [0]), p, 1, y2, N2, 1024, 1, None) == KATA_EINVAL


def test_fwht_rejects_aliasing():
    """An output overlapping an input is rejected before any launch (workgroups re-read their
    row while others write theirs); no GPU is needed for the argument checks."""
    import ctypes
    from kata_amd.capi import lib, KATA_EINVAL
    L = lib()
    buf = (ctypes.c_float * (4 * 1024 * 4 + 64))()
    base = (ctypes.addressof(buf) + 15) & ~15
    x, y, gs, out = base, base + 4096 * 4, base + 2 * 4096 * 4, base + 3 * 4096 * 4
    W, M = 1024, 4
    # xnew == x (in-place residual), xnew == y, out over x, out over gs
    for args in ((x, y, gs, out, x), (x, y, gs, out, y), (x, y, gs, x + 64, None), (x, y, gs, gs, None)):
        xx, yy, gg, oo, xn = args
        rc = L.kata_add_rms_fwht(xx, yy, gg, oo, 0, 0, xn, None, None, 0, W, M, None)
        assert rc == KATA_EINVAL and b"overlap" in L.kata_last_error(), args
    rc = L.kata_rms_fwht(x, y, gs, y, 0, 0, W, M, 1, None)       # out over src2 (SwiGLU)
    assert rc == KATA_EINVAL and b"overlap" in L.kata_last_error()


def test_torch_front_end_checks_sizes():
    """Shape arguments that do not match the tensors raise ValueError before anything
    reaches the device (CPU tensors: the size checks come first)."""
    import torch
    from kata_amd import ops
    W = torch.zeros(2 * 40 * 28, dtype=torch.uint8)            # 2 rows of K = 5120
    x = torch.zeros((1, 5120), dtype=torch.float16)
    with pytest.raises(ValueError, match="W holds"):
        ops.gemv_ptq1(W, x, 5120, 3)                            # N too large for W
    with pytest.raises(ValueError, match="x holds"):
        ops.gemv_ptq1(W, x, 5120, 2, T=2)                       # x has one token
    with pytest.raises(ValueError, match="out holds"):
        ops.gemv_ptq1(W, x, 5120, 2, out=torch.zeros(1))
    with pytest.raises(ValueError, match="multiple"):
        ops.gemv_ptq1(W, x, 5000, 2)
    with pytest.raises(ValueError, match=r"Ws\[1\] holds"):
        ops.gemv_ptq1_batch([W, W[:100]], x, 5120, [2, 2])
    with pytest.raises(ValueError, match="W holds"):
        ops.gemv_q8(torch.zeros(10, dtype=torch.uint8), x, 5120, 1)
    with pytest.raises(ValueError, match="lda"):
        ops.gemm_ptq1_f16(torch.zeros((4, 1024), dtype=torch.float16), W, 5120, 2)
    with pytest.raises(ValueError, match="SX"):
        ops.gemm_ptq1_i8(torch.zeros((4, 5120), dtype=torch.int8), torch.zeros((40, 2)), W, 5120, 2)
    with pytest.raises(ValueError, match="W holds"):
        ops.expand_f16(W, 5120, 3)


def test_gemv_operand_form_sizes_and_rejects():
    """Sizes of the decode GEMV's operand form (image 256 T B per block over nq even steps of
    4 blocks, then 8 B scale pairs per block and token) and the argument checks of its
    producers and consumers, before any launch."""
    lib = L.lib()
    nq = lambda K: ((K // 128 + 3) // 4 + 1) & ~1
    for K, T in ((128, 1), (1152, 2), (5120, 1), (5120, 2), (17408, 1), (17408, 2)):
        assert lib.kata_gemv_xq_bytes(K, T) == nq(K) * T * (1024 + 32)
    for K, T in ((5120, 3), (17408, 8), (128, 5)):                       # the wide GEMV's image
        assert lib.kata_gemv_xq_bytes(K, T) == K // 128 * (2048 + 32)
    assert lib.kata_gemv_xq_bytes(5120, 9) == 0 and lib.kata_gemv_xq_bytes(100, 1) == 0
    assert lib.kata_gemv_xq_bytes(0, 1) == 0
    big = lib.kata_gemv_ptq1_max_k(1) + 128
    assert lib.kata_gemv_xq_bytes(big, 1) == 0
    prep = lib.kata_gemv_prepare_x
    out = ctypes.c_void_p(0x20000)
    assert prep(FAKE, 1, 0, 5120, 9, out, None) == KATA_EINVAL          # T
    assert prep(FAKE, 1, 1, 5120, 3, out, None) == KATA_EINVAL          # half2 only for T = 2
    assert prep(FAKE, 1, 0, 5000, 1, out, None) == KATA_EINVAL          # K % 128
    assert prep(FAKE, 2, 0, 5120, 1, out, None) == KATA_EINVAL          # x dtype (not itself)
    assert prep(FAKE, 0, 1, 5120, 2, out, None) == KATA_EINVAL          # half2 needs fp16
    assert prep(FAKE, 1, 0, 5120, 1, ctypes.c_void_p(0x20008), None) == KATA_EINVAL   # alignment
    assert prep(FAKE, 1, 0, 5120, 1, ctypes.c_void_p(0x10000 + 4096), None) == KATA_EINVAL   # overlap
    assert prep(None, 1, 0, 5120, 1, out, None) == KATA_EINVAL
    gemv = lib.kata_gemv_ptq1
    assert gemv(FAKE, out, 2, 1, FAKE, 5120, 64, 2, None) == KATA_EINVAL   # operand form: rows only
    # transforms: the operand form takes M <= 2 and the rows layout
    fwht = lib.kata_rms_fwht
    g = ctypes.c_void_p(0x40000)
    assert fwht(FAKE, None, g, out, 2, 0, 5120, 9, 3, None) == KATA_EINVAL
    assert fwht(FAKE, None, g, out, 2, 1, 5120, 2, 3, None) == KATA_EINVAL
