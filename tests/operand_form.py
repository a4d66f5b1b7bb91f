"""Reading the GEMVs' operand form (KATA_XQ) back on the host, for the tests: the documented
layouts decoded to x = s * (256 hi + lo).  T <= 2 (decode GEMV): per block A rows
[m 2][g 4][2 t + limb][16 B], element e at the byte given by the dense operand map, blocks
quarter-major over nq steps of 4, then (s, 0) fp32 pairs per block and token.  T = 3..8 (wide
GEMV): per block [m 2][g 4][row 16][16 B] (rows of tokens >= T zero), then per block the
scales of the 8 token slots (zero past T)."""
import numpy as np


def _elem_src(e):
    """(byte p, digit n) of element e of a PTQ1_0 block (shaders/common.h:13-17)."""
    if e < 80:
        return e & 15, e >> 4
    if e < 120:
        return 16 + ((e - 80) & 7), (e - 80) >> 3
    return 24 + ((e - 120) & 1), (e - 120) >> 1


def img_off(e, T):
    """Byte of element e in a block's A image: lane group g holds qs bytes 6g..6g+5 and two
    qh digits; MFMA m=0 takes digits 1..4 of the first four bytes, m=1 the rest."""
    p, n = _elem_src(e)
    if p < 24:
        g, j = p // 6, p % 6
        if n > 0:
            m, slot = (0 if j < 4 else 1), 4 * (j & 3) + n - 1
        else:
            m, slot = 1, 8 + j
    else:
        g, m, slot = 2 * (p - 24) + (n >> 1), 1, 14 + (n & 1)
    return m * (4 * 2 * T * 16) + g * (2 * T * 16) + slot


def decode_wide(xq, K, T):
    """x[t][k] back from the wide operand form (T = 3..8); checks the rows past T are zero."""
    xq = np.asarray(xq, dtype=np.uint8)
    nb = K // 128
    sc = xq[nb * 2048:nb * 2048 + nb * 32].view(np.float32).reshape(nb, 8)
    assert not sc[:, T:].any()
    offs = np.array([img_off(e, 8) for e in range(128)])
    x = np.zeros((T, K), np.float64)
    for b in range(nb):
        blk = xq[b * 2048:(b + 1) * 2048]
        rows = blk.reshape(2, 4, 16, 16)
        assert not rows[:, :, 2 * T:, :].any()
        for t in range(T):
            hi = blk[offs + 32 * t].view(np.int8).astype(np.int64)
            lo = blk[offs + 32 * t + 16].view(np.int8).astype(np.int64)
            x[t, 128 * b:128 * b + 128] = sc[b, t] * (256 * hi + lo)
    return x


def decode(xq, K, T):
    """x[t][k] (float64) back from the operand form's bytes; checks the zero padding."""
    if T > 2:
        return decode_wide(xq, K, T)
    xq = np.asarray(xq, dtype=np.uint8)
    nb, nq = K // 128, ((K // 128 + 3) // 4 + 1) & ~1
    blk = 256 * T
    qbytes = nq * blk
    sc = xq[4 * qbytes:4 * qbytes + 8 * 4 * nq * T].view(np.float32).reshape(4 * nq, T, 2)
    assert np.all(sc[:, :, 1] == 0)
    offs = np.array([img_off(e, T) for e in range(128)])
    x = np.zeros((T, K), np.float64)
    for b in range(nb):
        base = (b & 3) * qbytes + (b >> 2) * blk
        for t in range(T):
            hi = xq[base + offs + 32 * t].view(np.int8).astype(np.int64)
            lo = xq[base + offs + 32 * t + 16].view(np.int8).astype(np.int64)   # q - 256 hi, signed
            x[t, 128 * b:128 * b + 128] = sc[b, t, 0] * (256 * hi + lo)
    for b in range(nb, 4 * nq):                      # zero padding blocks
        base = (b & 3) * qbytes + (b >> 2) * blk
        assert not xq[base:base + blk].any() and not sc[b].any()
    return x


def nbytes(K, T):
    if T > 2:
        return K // 128 * (2048 + 32)
    nq = ((K // 128 + 3) // 4 + 1) & ~1
    return nq * T * (1024 + 32)


def bound_ok(xd, x, extra=0.0):
    """|xd - x| within the block quantiser's bound amax / 65278 (1 % slack for the fp32
    rounding of x * 32639 / amax) plus `extra`, per 128-block and token."""
    T, K = x.shape
    amax = np.abs(x).reshape(T, K // 128, 128).max(axis=2, keepdims=True)
    err = np.abs(xd - x).reshape(T, K // 128, 128)
    return bool(np.all(err <= amax * (1.01 / 65278) + extra + 1e-30))
