"""Pins the CPU oracle (oracle/kata_oracle.c) before it is trusted as the parity checker.

Each check is chosen so that a plausible slip (wrong digit order, transposed element
map, off-by-one in the ceil packing, dropped scale, wrong rounding mode) fails:
closed forms, exhaustive tables, round trips, brute force on small shapes, and the
independently generated fixtures in tests/golden/.
"""
import numpy as np
import pytest

from oracle import oracle as orc


# ------------------------------------------------------------------ fp16 conversions
def test_half_to_float_all_patterns():
    L = orc.lib()
    pats = np.arange(65536, dtype=np.uint16)
    ref = pats.view(np.float16).astype(np.float32)
    got = np.array([L.orc_half_to_float(int(p)) for p in pats], np.float32)
    finite = np.isfinite(ref)
    assert np.array_equal(got[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(ref)]))


def test_float_to_half_rne():
    L = orc.lib()
    rng = np.random.default_rng(1)
    vals = np.concatenate([
        rng.standard_normal(4000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 5, 4000),
        # exact ties between neighbouring halves
        ((np.arange(1, 2000, dtype=np.float32) + np.float32(0.5)) * np.float32(2.0 ** -10)),
        np.array([0.0, -0.0, 65504.0, 65520.0, 6.0e-8, 2.0 ** -25, 3 * 2.0 ** -26], np.float32),
    ]).astype(np.float32)
    got = np.array([L.orc_float_to_half(float(v)) for v in vals], np.uint16)
    ref = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


# ------------------------------------------------------------------ digits and element map
def test_digit_exhaustive_closed_form(golden):
    tab = golden["digit_table"]
    for b in range(256):
        for n in range(5):
            want = (b * 3 ** (n + 1) // 256) % 3
            assert tab[b, n] == want
            assert orc.digit(b, n) == want
            assert orc.lib().orc_ptq1_digit_float(b, n) == want


def test_base3_round_trip_all_tuples():
    # every 5-digit tuple -> ceil(q*256/243) -> digits back (qs bytes)
    for q in range(243):
        b = -((-q * 256) // 243)
        digs = [(q // 3 ** (4 - n)) % 3 for n in range(5)]
        assert [orc.digit(b, n) for n in range(5)] == digs
    # every 4-digit tuple, shifted by one digit (qh bytes)
    for q4 in range(81):
        b = -((-(3 * q4) * 256) // 243)
        digs = [(q4 // 3 ** (3 - n)) % 3 for n in range(4)]
        assert [orc.digit(b, n) for n in range(4)] == digs
        assert orc.digit(b, 4) == 0


def test_element_map_vs_spec_and_loop(golden):
    rng = np.random.default_rng(2)
    for _ in range(20):
        blk = rng.integers(0, 256, 28, dtype=np.uint8)
        blk[26:28] = np.array([np.float16(0.75)]).view(np.uint8)
        loop = np.empty(128, np.float32)
        orc.lib().orc_ptq1_dequant_row(orc._p(blk), orc._p(loop), 128)
        for e in range(128):
            p, n = int(golden["elem_byte"][e]), int(golden["elem_digit"][e])
            want = (int(blk[p]) * 3 ** (n + 1) // 256) % 3 - 1
            assert orc.lib().orc_ptq1_elem_trit(orc._p(blk), e) == want
            assert loop[e] == np.float32(want * 0.75)


def test_single_hot_elements():
    # a +1 at element e (all others 0) must land exactly at e after pack -> decode
    for e in range(128):
        t = np.zeros((1, 128), np.int8); t[0, e] = 1
        W = orc.pack(t, np.array([[1.0]], np.float16))
        deq = orc.dequant(W, 128, 1)
        assert deq[0, e] == 1.0 and np.count_nonzero(deq) == 1


# ------------------------------------------------------------------ packing / quantiser
def test_pack_matches_golden(golden):
    W = orc.pack(golden["ptq1_trits"], golden["ptq1_scales"])
    assert np.array_equal(W, golden["ptq1_W"])


def test_dequant_matches_golden(golden):
    K, N = int(golden["ptq1_K"]), int(golden["ptq1_N"])
    deq = orc.dequant(golden["ptq1_W"], K, N)
    assert np.array_equal(deq.astype(np.float64), golden["ptq1_deq"])


def test_quantiser_round_trip():
    rng = np.random.default_rng(3)
    N, K = 16, 512
    t = rng.integers(-1, 2, (N, K)).astype(np.int8)
    t[:, ::128] = 1     # amax = d exactly in each block
    d = np.abs(rng.normal(0, 0.02, (N, K // 128))).astype(np.float16).astype(np.float32)
    X = (t.astype(np.float32).reshape(N, K // 128, 128) * d[:, :, None]).reshape(N, K)
    Wq = orc.quantize(X)
    Wp = orc.pack(t, d.astype(np.float16))
    assert np.array_equal(Wq, Wp)
    assert np.array_equal(orc.dequant(Wq, K, N), X)


def test_quantiser_rounding_thresholds():
    # lroundf(x/d): |x| < d/2 -> 0, |x| >= d/2 -> +-1 (half away from zero)
    x = np.zeros((1, 128), np.float32)
    x[0, 0] = 2.0
    x[0, 1] = 0.999
    x[0, 2] = 1.0
    x[0, 3] = -1.0
    x[0, 4] = -0.999
    W = orc.quantize(x)
    deq = orc.dequant(W, 128, 1)[0] / 2.0
    assert list(deq[:5]) == [1.0, 0.0, 1.0, -1.0, 0.0]


# ------------------------------------------------------------------ GEMV oracles
def test_gemv_golden(golden):
    K, N = int(golden["ptq1_K"]), int(golden["ptq1_N"])
    x = golden["gemv_x"].astype(np.float32)
    y = orc.gemv_ptq1(golden["ptq1_W"], x, K, N, 2)
    np.testing.assert_allclose(y, golden["gemv_y"], rtol=1e-12, atol=1e-12)


def test_gemv_special_cases(golden):
    K, N = int(golden["ptq1_K"]), int(golden["ptq1_N"])
    W, t, s = golden["ptq1_W"], golden["ptq1_trits"], golden["ptq1_scales"].astype(np.float64)
    x = golden["gemv_x"].astype(np.float32)
    y = orc.gemv_ptq1(W, x, K, N, 2)
    assert y[0, 5] == 0.0                                  # all-zero trits
    assert y[0, 7] == pytest.approx(s[7, 0] * x[0, 123])   # single hot element -> d * x[e]
    assert y[0, 8] == pytest.approx(-s[8, 0] * x[0, 87])
    # x = 1 -> sum_b d_b * sum(t_b)
    want = (t.reshape(N, K // 128, 128).sum(-1) * s).sum(-1)
    np.testing.assert_allclose(y[1], want, rtol=1e-12)


def test_gemv_brute_force_random():
    rng = np.random.default_rng(4)
    for K, N, T in [(128, 3, 1), (384, 17, 2), (1024, 8, 2)]:
        W, t, s = orc.synth_ptq1(N, K, seed=int(rng.integers(1 << 30)))
        x = rng.standard_normal((T, K)).astype(np.float32)
        deq = (t.reshape(N, K // 128, 128) * s.astype(np.float64)[:, :, None]).reshape(N, K)
        want = x.astype(np.float64) @ deq.T
        np.testing.assert_allclose(orc.gemv_ptq1(W, x, K, N, T), want, rtol=1e-10, atol=1e-10)


def test_q8_golden(golden):
    y = orc.gemv_q8(golden["q8_W"], golden["q8_x"].astype(np.float32), 64, 8, 2)
    np.testing.assert_allclose(y, golden["q8_y"], rtol=1e-12, atol=1e-14)


def test_q8_brute_force():
    W, q, s = orc.synth_q8(5, 256, seed=9)
    x = orc.synth_x(2, 256, seed=10).astype(np.float32)
    deq = (q.reshape(5, 8, 32).astype(np.float64) * s.astype(np.float64)[:, :, None]).reshape(5, 256)
    np.testing.assert_allclose(orc.gemv_q8(W, x, 256, 5, 2), x.astype(np.float64) @ deq.T, rtol=1e-10)


def test_cpu_baseline_matches_oracle():
    W, _, _ = orc.synth_ptq1(64, 1024, seed=11)
    x = orc.synth_x(2, 1024, seed=12).astype(np.float32)
    ref = orc.gemv_ptq1(W, x, 1024, 64, 2)
    got = orc.cpu_gemv_f32(W, x, 1024, 64, 2, 0, 64, 2)
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) < 1e-5
    got = orc.cpu_gemv_stage(W, x, 1024, 64, 2, 0, 64, 2)     # the reference's host form
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) < 1e-5


# ------------------------------------------------------------------ prefill oracles
def test_expand_f16_golden(golden):
    K, N = int(golden["ptq1_K"]), int(golden["ptq1_N"])
    e = orc.expand_f16(golden["ptq1_W"], K, N)
    assert np.array_equal(e.view(np.uint16), golden["expand_f16"].view(np.uint16))


def test_gemm_f16_golden(golden):
    K, N = int(golden["ptq1_K"]), int(golden["ptq1_N"])
    C = orc.gemm_f16(golden["gemm_A"], golden["ptq1_W"], 5, K, N)
    np.testing.assert_allclose(C, golden["gemm_C"], rtol=1e-12, atol=1e-12)


def test_quant_rows_golden(golden):
    Q, SX = orc.quant_rows(golden["qr_X"], 3, 256)
    assert np.array_equal(Q, golden["qr_Q"])
    assert np.array_equal(SX.view(np.uint32), golden["qr_SX"].view(np.uint32))
    # all-zero group -> scale 1, codes 0 ; ties round to even
    assert SX[1, 1] == 1.0 and not Q[1, 128:].any()
    assert list(Q[2, :4]) == [127, 0, 2, -2]


def test_expand_i8_and_gemm_i8_golden(golden):
    K, N = int(golden["ptq1_K"]), int(golden["ptq1_N"])
    T8, SW = orc.expand_i8(golden["ptq1_W"], K, N)
    assert np.array_equal(T8, golden["ptq1_trits"])
    assert np.array_equal(SW, golden["ptq1_scales"].astype(np.float32))
    C, GS = orc.gemm_i8(golden["qr_Q"], golden["qr_SX"], golden["ptq1_W"], 3, K, N, want_group_sums=True)
    assert np.array_equal(GS, golden["i8_GS"])
    want = (GS.astype(np.float64) * SW.astype(np.float64)[None, :, :]
            * golden["qr_SX"].T.astype(np.float64)[:, None, :]).sum(-1)
    np.testing.assert_allclose(C, want, rtol=1e-6, atol=1e-7)


def test_cpu_baseline_gemm_matches_oracle_gemm():
    """The bench's CPU GEMM baseline (fp32, tiled over weight rows) computes the same
    products as the double-precision oracle GEMM, on a ragged row count."""
    M, K, N = 37, 640, 23
    W, _, _ = orc.synth_ptq1(N, K, 71)
    A = orc.synth_x(M, K, 72)
    C = orc.cpu_gemm_f32(A, W, M, K, N, 0, N, 2)
    R = orc.gemm_f16(A, W, M, K, N)
    assert np.abs(C - R).max() <= 1e-5 * np.abs(R).max()


# ----------------------------------------------------------------------------- matmul input transform
def test_norm_fwht_plain_matches_hadamard_matrix():
    """Mode 3 (u = src * gs) against the Sylvester Hadamard matrix (scipy.linalg.hadamard,
    natural order: H[j][k] = (-1)^popcount(j & k)) applied per 1024-block, / 32."""
    from scipy.linalg import hadamard
    H = hadamard(1024).astype(np.float64)
    rng = np.random.default_rng(5)
    src = rng.standard_normal((3, 2048)).astype(np.float32)
    gs = rng.choice([-1.0, 1.0], size=2048).astype(np.float32)
    out, _ = orc.norm_fwht(src, gs, 3)
    u = src.astype(np.float64) * gs
    ref = np.concatenate([u[:, :1024] @ H.T, u[:, 1024:] @ H.T], axis=1) / 32.0
    assert np.abs(out - ref).max() < 1e-9 * np.abs(ref).max()


def test_norm_fwht_involution_and_rms_closed_form():
    """(H/32)^2 = I: transforming the transform with gs = 1 returns the input; mode 0 with a
    constant row c gives inv = 1/sqrt(c^2 + 1e-6), so H of v*inv*gs is checked on a row whose
    transform is known: a constant block maps to 32 * c * inv at j = 0 and 0 elsewhere."""
    rng = np.random.default_rng(6)
    src = rng.standard_normal((2, 1024)).astype(np.float32)
    ones = np.ones(1024, np.float32)
    once, _ = orc.norm_fwht(src, ones, 3)
    twice, _ = orc.norm_fwht(once.astype(np.float32), ones, 3)
    assert np.abs(twice - src).max() < 1e-5
    c = 0.75
    x = np.full((1, 1024), c, np.float32)
    out, hout = orc.norm_fwht(x, ones, 0, gamma=np.full(1024, 2.0, np.float32))
    inv = 1.0 / np.sqrt(c * c + 1e-6)
    assert abs(out[0, 0] - 32.0 * c * inv) < 1e-9 and np.abs(out[0, 1:]).max() < 1e-12
    assert np.allclose(hout, 2.0 * c * inv, rtol=1e-12)
    # residual add: x + y with y = -x + c gives the same constant row
    y = (c - src[:1]).astype(np.float32)
    out2, _ = orc.norm_fwht(src[:1], ones, 0, src2=y, add=True)
    assert abs(out2[0, 0] - 32.0 * c * inv) < 1e-5


def test_norm_fwht_swiglu_and_gdn_order():
    """Mode 1 is silu(a) * b (checked with H applied twice, back to the elementwise value);
    mode 2 reads src[h + 128 (t/3 + 16 (t%3))] for i = 128 t + h, a permutation of 6144."""
    rng = np.random.default_rng(7)
    a = rng.standard_normal((1, 1024)).astype(np.float32)
    b = rng.standard_normal((1, 1024)).astype(np.float32)
    ones = np.ones(1024, np.float32)
    out, _ = orc.norm_fwht(a, ones, 1, src2=b)
    back, _ = orc.norm_fwht(out.astype(np.float32), ones, 3)
    ref = a.astype(np.float64) / (1.0 + np.exp(-a.astype(np.float64))) * b
    assert np.abs(back - ref).max() < 1e-5
    i = np.arange(6144)
    h, t = i & 127, i >> 7
    perm = h + 128 * (t // 3 + 16 * (t % 3))
    assert np.array_equal(np.sort(perm), i)
    src = np.arange(6144, dtype=np.float32)[None, :]
    ones6 = np.ones(6144, np.float32)
    out, _ = orc.norm_fwht(src, ones6, 2)
    back = np.concatenate([orc.norm_fwht(out[:, 1024 * k:1024 * (k + 1)].astype(np.float32), ones, 3)[0]
                           for k in range(6)], axis=1)
    assert np.abs(back[0] - perm).max() < 1e-3


def test_float_pipe_identity_exhaustive(golden):
    """The reference's float-pipe decode (shaders/gemv_fast.metal:2-3): with u = b / 256 and
    g_k = floor(3^k u), digit n = g_{n+1} - 3 g_n, evaluated in fp32 (exact: 3^5 * 255 =
    61965 < 2^24), equals the integer digit for all 256 bytes x 5 digits; and its
    coefficient form sum_n t_n y_n = sum_{k=1..4} g_k (y_{k-1} - 3 y_k) + g_5 y_4 holds."""
    b = np.arange(256, dtype=np.float32)
    u = b / np.float32(256.0)
    g = [np.floor(np.float32(3.0 ** k) * u) for k in range(6)]
    digits = np.stack([g[n + 1] - 3 * g[n] for n in range(5)], axis=1).astype(np.int64)
    assert np.array_equal(digits, golden["digit_table"].astype(np.int64))
    assert np.array_equal(digits, np.array([[orc.digit(int(v), n) for n in range(5)] for v in range(256)]))
    y = np.random.default_rng(0).standard_normal((256, 5))
    lhs = (digits * y).sum(axis=1)
    rhs = sum(g[k].astype(np.float64) * (y[:, k - 1] - 3 * y[:, k]) for k in range(1, 5)) + g[5] * y[:, 4]
    assert np.allclose(lhs, rhs, rtol=0, atol=1e-12)


def test_expand_q8_matches_numpy():
    """k_expand_q8: half(d * q) rounded to nearest even, incl. subnormal results and
    overflow to infinity, bit for bit against numpy's float32 -> float16 conversion."""
    rng = np.random.default_rng(21)
    N, K = 6, 128
    q = rng.integers(-128, 128, size=(N, K), dtype=np.int64).astype(np.int8)
    d = (rng.choice([1e-7, 3e-5, 0.02, 1.0, 300.0, 700.0], size=(N, K // 32)) *
         rng.choice([-1.0, 1.0], size=(N, K // 32))).astype(np.float16)
    W = orc.q8_pack(q, d)
    got = orc.expand_q8_f16(W, K, N)
    with np.errstate(over="ignore"):
        ref = (np.repeat(d.astype(np.float32), 32, axis=1) * q.astype(np.float32)).astype(np.float16)
    assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))
    assert np.isinf(got).any() and (np.abs(got[np.isfinite(got)]) < 6.1e-5).any()


def test_gemm_q8_oracle_vs_numpy():
    W, q, d = orc.synth_q8(9, 256, 22)
    A = orc.synth_x(5, 256, 23)
    wexp = orc.expand_q8_f16(W, 256, 9).astype(np.float64)
    np.testing.assert_allclose(orc.gemm_q8_f16(A, W, 5, 256, 9), A.astype(np.float64) @ wexp.T, rtol=1e-12, atol=1e-12)
