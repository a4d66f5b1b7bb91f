"""GPU parity of the sublayer matmul halves (kata_dispatch_in / kata_dispatch_out) at the 27B
shapes of the two mixers, against the oracle's composition of the same steps:

  GDN (src/engine.cpp:150-160): h = H(rmsnorm(x + y) * gs), qkv (10240) and z (6144) of h;
      out = ssm_out(H(head-ordered o * gs_o)), o 6144 wide (mode 2).
  GQA (src/engine.cpp:161-175): h as above, q (12288), k and v (1024) of h;
      out = wo(H(o * gs_o)), o 6144 wide (mode 3).

Each form is checked step by step from the work buffer (the transformed activation the
entry point leaves at its start: fp32 [K] decode, fp16 [M][K] prefill and verify), the
matmuls on sampled weight rows against the oracle fed with that activation, then the
transform against the oracle's double-precision transform.  Bars: decode and verify
GEMVs 2e-4 relative L2 (16-bit block activations), prefill GEMMs 1e-5 (exact fp16 and
int8 arithmetic with fp32 accumulation), the fp16 activation within one fp16 ulp of the
largest element, the residual x + y bit-exact."""
import numpy as np
import pytest
import torch

from kata_amd.engine import Dispatch, dispatch_work_bytes
from oracle import oracle as orc
from tests import operand_form
from tests.conftest import rel_l2

pytestmark = pytest.mark.gpu
H = 5120
MIXERS = {
    "gdn": dict(ins=[("qkv", 10240), ("z", 6144)], out=("ssmout", 6144, 2)),
    "gqa": dict(ins=[("wq", 12288), ("wk", 1024), ("wv", 1024)], out=("wo", 6144, 3)),
}
ROWS = 97          # every 97th weight row goes through the oracle


def _signs(W, seed):
    rng = np.random.default_rng(seed)
    return (rng.choice([-1.0, 1.0], W) * rng.uniform(0.5, 1.5, W)).astype(np.float32)


def _weights(mix, seed):
    spec = MIXERS[mix]
    mats, parts, offs, o = {}, [], {}, 0
    shapes = [(nm, N, H) for nm, N in spec["ins"]] + [(spec["out"][0], H, spec["out"][1])]
    for i, (nm, N, K) in enumerate(shapes):
        W, _, _ = orc.synth_ptq1(N, K, seed + i)
        pad = np.zeros(36, np.uint8)          # offsets that are not multiples of 16
        parts += [pad, W.ravel()]
        o += pad.size
        offs[nm] = o
        o += W.size
        mats[nm] = W
    return np.concatenate(parts), offs, mats


@pytest.fixture(scope="module", params=["gdn", "gqa"])
def mixer(request):
    dev = torch.device("cuda:0")
    buf, offs, mats = _weights(request.param, 900 if request.param == "gdn" else 950)
    d = Dispatch(torch.from_numpy(buf).to(dev))
    return request.param, d, offs, mats


def _mm_ref(form, W, A, K, i8):
    """The oracle's matmul of activation rows A [M][K] with the sampled rows of W."""
    rows = np.arange(0, W.shape[0], ROWS)
    Ws = np.ascontiguousarray(W[rows])
    M = A.shape[0]
    if form != "prefill":
        return orc.gemv_ptq1(Ws, A.astype(np.float32), K, len(rows), M), rows
    if i8:
        Q, SX = orc.quant_rows(A, M, K)
        return orc.gemm_i8(Q, SX, Ws, M, K, len(rows)), rows
    return orc.gemm_f16(A, Ws, M, K, len(rows)), rows


def _act(work, form, K, M):
    """The transformed activation in the work buffer: the decode and verify forms hold the
    GEMVs' operand form (decoded here), the prefill form fp16 rows."""
    wk = work.cpu().numpy()
    if form != "prefill":
        return operand_form.decode(wk[:operand_form.nbytes(K, M)], K, M)
    return wk[:2 * M * K].view(np.float16).reshape(M, K)


def _act_ok(a, ref, form):
    """Transform output: fp16 rows within 2^-11 of the reference's max; the operand form
    within its block quantiser's bound plus 1e-5 of the max (the fp32 transform)."""
    if form == "prefill":
        return np.abs(a.astype(np.float64) - ref).max() <= np.abs(ref).max() * 2.0 ** -11
    return operand_form.bound_ok(a, ref, np.abs(ref).max() * 1e-5)


@pytest.mark.parametrize("form,M,i8", [("decode", 1, "none"), ("prefill", 24, "none"), ("prefill", 24, "all"),
                                       ("verify", 1, "none"), ("verify", 3, "none"), ("verify", 8, "none")])
def test_sub_in_out(mixer, form, M, i8):
    mix, d, offs, mats = mixer
    d.set_i8(i8)
    dev = torch.device("cuda:0")
    spec = MIXERS[mix]
    rng = np.random.default_rng([len(mix), M, len(form), len(i8)])
    x = rng.standard_normal((M, H)).astype(np.float32)
    y = (0.3 * rng.standard_normal((M, H))).astype(np.float32)
    gs = _signs(H, 5)
    Tt = lambda a: torch.from_numpy(a).to(dev)
    tol = 1e-5 if form == "prefill" else 2e-4

    # input half
    xnew = torch.empty((M, H), dtype=torch.float32, device=dev)
    work = torch.full((dispatch_work_bytes(form, H, M),), 0x7f, dtype=torch.uint8, device=dev)
    mats_in = [(offs[nm], N, nm) for nm, N in spec["ins"]]
    outs = d.sub_in(form, mats_in, Tt(x), Tt(y), Tt(gs), xnew=xnew, work=work)
    torch.cuda.synchronize()
    assert np.array_equal(xnew.cpu().numpy(), x + y)
    h = _act(work, form, H, M)
    h_ref, _ = orc.norm_fwht(x, gs, 0, src2=y, add=True)
    assert _act_ok(h, h_ref, form)
    for (nm, N), o in zip(spec["ins"], outs):
        ref, rows = _mm_ref(form, mats[nm], h, H, i8 == "all")
        e = rel_l2(o.cpu().numpy()[:, rows], ref)
        assert e.max() < tol, (mix, form, nm, e.max())

    # output half
    nm, W, mode = spec["out"]
    o = (0.5 * rng.standard_normal((M, W))).astype(np.float32)
    gso = _signs(W, 6)
    work = torch.full((dispatch_work_bytes(form, W, M),), 0x7f, dtype=torch.uint8, device=dev)
    out = d.sub_out(form, offs[nm], nm, Tt(o), None, mode, Tt(gso), H, work=work)
    torch.cuda.synchronize()
    t = _act(work, form, W, M)
    t_ref, _ = orc.norm_fwht(o, gso, mode)
    assert _act_ok(t, t_ref, form)
    ref, rows = _mm_ref(form, mats[nm], t, W, i8 == "all")
    e = rel_l2(out.cpu().numpy()[:, rows], ref)
    assert e.max() < tol, (mix, form, nm, e.max())


def test_sub_decode_is_the_gemv(mixer):
    """The decode input half equals the standalone transform + batched GEMV bit for bit."""
    from kata_amd import ops
    mix, d, offs, mats = mixer
    dev = torch.device("cuda:0")
    spec = MIXERS[mix]
    rng = np.random.default_rng(3)
    x = torch.from_numpy(rng.standard_normal((1, H)).astype(np.float32)).to(dev)
    gs = torch.from_numpy(_signs(H, 7)).to(dev)
    outs = d.sub_in("decode", [(offs[nm], N, nm) for nm, N in spec["ins"]], x, None, gs)
    h = ops.add_rms_fwht(x, gs)[0]
    for (nm, N), o in zip(spec["ins"], outs):
        W = torch.from_numpy(mats[nm]).to(dev)
        y1 = ops.gemv_ptq1(W, h, H, N, 1)
        torch.cuda.synchronize()
        assert torch.equal(o, y1), nm
