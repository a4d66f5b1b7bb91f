"""GGUF v3 reader of the C ABI on files written by tests/gguf_writer.py: tensor index,
offsets, sizes, metadata, malformed files; on the GPU the uploaded data region feeds the
GEMVs by offset."""
import numpy as np
import pytest
import torch

from kata_amd import capi as L
from kata_amd.gguf import GGML_F32, GGML_PTQ1_0, GGML_Q8_0, GgufFile
from oracle import oracle as orc

from conftest import rel_l2
from gguf_writer import write_gguf


def _model(tmp_path, alignment=64):
    W1, _, _ = orc.synth_ptq1(48, 512, 11)            # blk.0.ffn_gate: 48 rows of K=512
    W2, _, _ = orc.synth_ptq1(20, 1024, 12)           # blk.0.ffn_down
    rng = np.random.default_rng(13)
    q8 = rng.integers(-127, 128, size=(16, 64 // 32, 34)).astype(np.int8).view(np.uint8)
    q8[:, :, 0:2] = np.abs(rng.normal(0, 0.02, (16, 2))).astype(np.float16).view(np.uint8).reshape(16, 2, 2)
    norm = rng.standard_normal(512).astype(np.float32)
    kvs = [("general.architecture", 8, "qwen35"), ("general.alignment", 4, alignment),
           ("qwen35.embedding_length", 4, 5120), ("qwen35.block_count", 5, 64), ("flag", 7, True),
           ("tokenizer.ggml.tokens", 9, (8, ["a", "bb", "ccc"])), ("rope.scale", 6, 0.5),
           ("ids", 9, (5, [1, -2, 3])), ("big", 10, 1 << 40)]
    tensors = [("blk.0.ffn_gate.weight", [512, 48], GGML_PTQ1_0, W1.tobytes()),
               ("blk.0.attn_norm.weight", [512], GGML_F32, norm.tobytes()),
               ("blk.0.ffn_down.weight", [1024, 20], GGML_PTQ1_0, W2.tobytes()),
               ("mtp.q8.weight", [64, 16], GGML_Q8_0, q8.tobytes())]
    path = str(tmp_path / "m.gguf")
    head, offs = write_gguf(path, kvs, tensors, alignment)
    return path, head, offs, (W1, W2, q8, norm)


def test_gguf_index_and_metadata(tmp_path):
    path, head, offs, (W1, W2, q8, norm) = _model(tmp_path)
    with GgufFile(path) as g:
        t = g.tensors
        assert list(t) == ["blk.0.ffn_gate.weight", "blk.0.attn_norm.weight", "blk.0.ffn_down.weight", "mtp.q8.weight"]
        assert t["blk.0.ffn_gate.weight"] == {"type": GGML_PTQ1_0, "dims": [512, 48, 1, 1], "offset": offs[0],
                                              "nbytes": W1.nbytes}
        assert t["blk.0.attn_norm.weight"]["nbytes"] == 2048 and t["blk.0.attn_norm.weight"]["dims"] == [512, 1, 1, 1]
        assert t["blk.0.ffn_down.weight"]["offset"] == offs[2] and t["blk.0.ffn_down.weight"]["nbytes"] == W2.nbytes
        assert t["mtp.q8.weight"]["type"] == GGML_Q8_0 and t["mtp.q8.weight"]["nbytes"] == q8.nbytes
        assert all(v["offset"] % 64 == 0 for v in t.values())
        assert g.data_bytes == offs[3] + q8.nbytes
        assert g.get_int("qwen35.embedding_length") == 5120 and g.get_int("general.alignment") == 64
        assert g.get_int("qwen35.block_count") == 64 and g.get_int("flag") == 1 and g.get_int("big") == 1 << 40
        assert g.get_str("general.architecture") == "qwen35" and g.get_str("missing") is None
        with pytest.raises(KeyError):
            g.get_int("rope.scale")                   # floats are not integer metadata
        assert L.lib().kata_gguf_find(g._h, b"blk.0.ffn_down.weight") == 2
        assert L.lib().kata_gguf_find(g._h, b"nope") == L.KATA_EINVAL


def test_gguf_rejects_malformed_files(tmp_path):
    path, head, offs, _ = _model(tmp_path)
    raw = open(path, "rb").read()
    cases = {"magic": b"GGUX" + raw[4:], "version": raw[:4] + (2).to_bytes(4, "little") + raw[8:],
             "truncated_header": raw[:head // 2], "truncated_data": raw[:head + offs[2] + 10]}
    for name, data in cases.items():
        p = tmp_path / f"{name}.gguf"
        p.write_bytes(data)
        assert not L.lib().kata_gguf_open(str(p).encode()), name
        assert L.lib().kata_last_error()
    assert not L.lib().kata_gguf_open(str(tmp_path / "absent.gguf").encode())


@pytest.mark.gpu
def test_gguf_upload_feeds_gemv_by_offset(tmp_path):
    from kata_amd import ops
    from kata_amd.engine import Dispatch
    dev = torch.device("cuda:0")
    path, head, offs, (W1, W2, q8, norm) = _model(tmp_path)
    with GgufFile(path) as g:
        buf = g.upload(dev)
        t = g.tensors
    raw = open(path, "rb").read()
    assert np.array_equal(buf.cpu().numpy(), np.frombuffer(raw[head:], np.uint8))
    d = Dispatch(buf)
    for name, W, K, N in (("blk.0.ffn_gate.weight", W1, 512, 48), ("blk.0.ffn_down.weight", W2, 1024, 20)):
        x = torch.from_numpy(orc.synth_x(1, K, K, np.float32)).to(dev)
        y = torch.empty((1, N), dtype=torch.float32, device=dev)
        d.gemv(t[name]["offset"], x, y, K, N)
        assert rel_l2(y.cpu().numpy(), orc.gemv_ptq1(W, x.cpu().numpy(), K, N, 1)).max() < 2e-4
    o = t["mtp.q8.weight"]["offset"]
    xq = torch.from_numpy(orc.synth_x(1, 64, 3)).to(dev)
    yq = ops.gemv_q8(buf[o:o + q8.nbytes], xq, 64, 16, 1).cpu().numpy()
    assert rel_l2(yq, orc.gemv_q8(q8.reshape(16, -1), xq.cpu().numpy(), 64, 16, 1)).max() < 1e-5


def _raw(infos, data_len, alignment=32, pad_data=True):
    """A GGUF file with hand-written tensor infos [(name, dims, type, offset)] and data_len
    zero bytes of data (pad_data=False: the file ends right after the header, unpadded)."""
    import struct
    def s(x):
        b = x.encode()
        return struct.pack("<Q", len(b)) + b
    head = b"GGUF" + struct.pack("<IQQ", 3, len(infos), 1) + s("general.alignment") + struct.pack("<II", 4, alignment)
    for name, dims, typ, off in infos:
        head += s(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", typ, off)
    if pad_data:
        head += b"\0" * ((-len(head)) % alignment)
    return head + b"\0" * data_len


def test_gguf_rejects_out_of_range_and_unknown(tmp_path):
    """Tensor ranges checked term by term (no uint64 wrap-around), unknown ggml types and
    element counts that overflow or are not whole blocks rejected, a header that runs past
    the end of the file rejected."""
    ok = _raw([("w", [256, 2], GGML_PTQ1_0, 0)], 112)
    p = tmp_path / "ok.gguf"
    p.write_bytes(ok)
    h = L.lib().kata_gguf_open(str(p).encode())
    assert h
    L.lib().kata_gguf_close(h)
    cases = {
        "wrapped_offset": _raw([("w", [256, 2], GGML_PTQ1_0, (1 << 64) - 64)], 112),
        "offset_past_end": _raw([("w", [256, 2], GGML_PTQ1_0, 64)], 112),
        "bytes_past_end": _raw([("w", [256, 2], GGML_PTQ1_0, 0)], 100),
        "unknown_type": _raw([("w", [256, 2], 99, 0)], 112),
        "dims_overflow": _raw([("w", [1 << 40, 1 << 40], GGML_F32, 0)], 64),
        "bytes_overflow": _raw([("w", [1 << 62, 1], GGML_F32, 0)], 64),
        "not_whole_blocks": _raw([("w", [100, 2], GGML_PTQ1_0, 0)], 112),
        "header_past_end": _raw([], 0, alignment=1 << 20, pad_data=False),
    }
    for name, data in cases.items():
        q = tmp_path / f"{name}.gguf"
        q.write_bytes(data)
        assert not L.lib().kata_gguf_open(str(q).encode()), name
        assert L.lib().kata_last_error(), name
