"""GGUF reading and writing (dwim_amd/gguf.py), on the CPU: the reference's
own round-trip test (inference/gguf.rs:322-376), the header bytes of a small
file written out by hand from the format's definition (model/gguf.rs:1-10,
inference/gguf.rs:1-12), the file blocks of each weight format against the
oracle's dequantizers, and the synthetic qwen35 writer against the names and
keys the reference loader reads.  The GPU test uploads matrices read from a
file and multiplies with them."""
import struct

import numpy as np
import pytest

import oracle as O
from dwim_amd import device as D
from dwim_amd import gguf as G
from dwim_amd import model as M


def test_reads_back_what_it_wrote(tmp_path):
    """inference/gguf.rs:326-375, the same file and checks."""
    path = str(tmp_path / "test.gguf")
    meta = [("general.architecture", G.string("qwen35")), ("qwen35.block_count", G.u32(2)),
            ("list", G.array([G.Value(G.I32, -1), G.Value(G.I32, 1)])), ("scale", G.f32(0.5))]
    f32s = np.array([1.0, 2.0, 3.0], np.float32).tobytes()
    bf16 = (np.arange(8, dtype=np.uint16) << 8).tobytes()
    G.write(path, meta, [("norm", (3,), G.F32, f32s), ("w", (4, 2), G.BF16, bf16)])
    g = G.Gguf(path)
    assert g.str("general.architecture") == "qwen35"
    assert g.u32("qwen35.block_count") == 2
    assert g.f32("scale") == 0.5
    assert g.array("list")[0].as_int() == -1
    with pytest.raises(G.GgufError):
        g.u32("missing")
    assert list(g.f32s("norm")) == [1.0, 2.0, 3.0]
    w = g.matrix("w")
    assert (w.fmt, w.shape) == (D.BF16, (2, 4))
    assert w.quants[3] == 3 << 8
    with pytest.raises(G.GgufError):
        g.matrix("norm")


def test_header_bytes_follow_the_format(tmp_path):
    """One key and one tensor, the bytes spelled out from the format: magic,
    version 3, counts, a u64-length string, a type id and value; the tensor's
    name, dimension count, dimensions innermost first, type and offset; zero
    padding to 32; the data."""
    path = str(tmp_path / "h.gguf")
    data = np.arange(32, dtype=np.float32).tobytes()
    G.write(path, [("a", G.u32(7))], [("t", (8, 4), G.F32, data)])
    want = b"GGUF" + (3).to_bytes(4, "little") + (1).to_bytes(8, "little") + (1).to_bytes(8, "little")
    want += (1).to_bytes(8, "little") + b"a" + (4).to_bytes(4, "little") + (7).to_bytes(4, "little")
    want += (1).to_bytes(8, "little") + b"t" + (2).to_bytes(4, "little")
    want += (8).to_bytes(8, "little") + (4).to_bytes(8, "little") + (0).to_bytes(4, "little") + (0).to_bytes(8, "little")
    want += bytes(-len(want) % 32) + data
    assert open(path, "rb").read() == want
    g = G.Gguf(path)
    assert g.data_start == len(want) - len(data)
    assert g.info("t").dims == (8, 4)


def test_every_metadata_type_round_trips(tmp_path):
    path = str(tmp_path / "m.gguf")
    vals = [G.Value(G.U8, 250), G.Value(G.I8, -5), G.Value(G.U16, 65000), G.Value(G.I16, -300),
            G.Value(G.U32, 4_000_000_000), G.Value(G.I32, -7), G.Value(G.F32V, 1.5), G.Value(G.BOOL, True),
            G.Value(G.STR, "naïve"), G.Value(G.U64, 1 << 40), G.Value(G.I64, -(1 << 40)), G.Value(G.F64, 0.1),
            G.array([G.string("x"), G.string("yz")])]
    G.write(path, [(f"k{i}", v) for i, v in enumerate(vals)], [])
    g = G.Gguf(path)
    for i, v in enumerate(vals):
        assert g.meta[f"k{i}"] == v
    with pytest.raises(G.GgufError):
        g.u32("k1")  # negative
    with pytest.raises(G.GgufError):
        g.str("k0")


def test_bad_files_are_refused(tmp_path):
    p = tmp_path / "bad.gguf"
    p.write_bytes(b"GGUF" + struct.pack("<IQQ", 2, 0, 0))
    with pytest.raises(G.GgufError, match="version 2"):
        G.Gguf(str(p))
    p.write_bytes(b"GGML" + bytes(20))
    with pytest.raises(G.GgufError, match="not a GGUF"):
        G.Gguf(str(p))
    # a tensor past the end of the file
    G.write(str(p), [], [("t", (32,), G.F32, bytes(128))])
    p.write_bytes(p.read_bytes()[:-64])
    with pytest.raises(G.GgufError, match="past the end"):
        G.Gguf(str(p)).bytes("t")
    with pytest.raises(G.GgufError, match="whole blocks"):
        G.row_bytes(G.Q4_K, 300)


def test_f32_matrices_round_to_bf16_to_nearest_even():
    """gpu/float.rs:32-36: ties go to the even bf16."""
    x = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 1.0 + 2 ** -9, -2.5, 3.0e38], np.float32)
    got = G.to_bf16(x)
    assert list(got) == [O.to_bf16(float(v)) for v in x]
    assert got[1] == 0x3F80 and got[2] == 0x3F82  # 1 + 2^-8 ties down to even, 1 + 3·2^-8 up to even


@pytest.mark.parametrize("fmt,gfmt", [(D.Q4_0, G.Q4_0), (D.Q8_0, G.Q8_0), (D.Q4_K, G.Q4_K), (D.Q6_K, G.Q6_K)])
def test_file_blocks_decode_as_the_format(tmp_path, fmt, gfmt):
    """The file's blocks of each format, read back as a device Tensor, decode
    (by the oracle's restatement of the reference's dequantizers) to what the
    host quantizer's Tensor decodes to; K-quant blocks pass unchanged."""
    rows, cols = 3, 512
    vals = O.Rng(11).floats(rows * cols).reshape(rows, cols)
    t = D.Tensor.quantize(fmt, vals)
    path = str(tmp_path / "q.gguf")
    G.write(path, [], [("m", (cols, rows), gfmt, G._file_blocks(t))])
    raw = bytes(G.Gguf(path).bytes("m"))
    assert len(raw) == rows * G.row_bytes(gfmt, cols)
    u = G.Gguf(path).matrix("m")
    assert (u.fmt, u.shape) == (fmt, (rows, cols))
    assert np.array_equal(u.quants, t.quants)
    if fmt in (D.Q4_0, D.Q8_0):
        assert np.array_equal(u.scales, t.scales)
    for r in range(rows):
        row = np.frombuffer(raw, np.uint8)[r * len(raw) // rows:(r + 1) * len(raw) // rows]
        if fmt == D.Q4_0:
            blocks = row.reshape(-1, 18)
            d = np.array([O.from_f16(int(b[0]) | int(b[1]) << 8) for b in blocks], np.float32)
            lo, hi = (blocks[:, 2:] & 0xF).astype(np.float32) - 8, (blocks[:, 2:] >> 4).astype(np.float32) - 8
            got = (np.concatenate([lo, hi], 1) * d[:, None]).ravel()
            want = O.dequantize_q4_0_row(t.scales[r * cols // 32:(r + 1) * cols // 32],
                                         t.quants[r * cols // 2:(r + 1) * cols // 2])
        elif fmt == D.Q8_0:
            blocks = row.reshape(-1, 34)
            d = np.array([O.from_f16(int(b[0]) | int(b[1]) << 8) for b in blocks], np.float32)
            got = (blocks[:, 2:].view(np.int8).astype(np.float32) * d[:, None]).ravel()
            want = O.dequantize_q8_0_row(t.scales[r * cols // 32:(r + 1) * cols // 32],
                                         t.quants[r * cols:(r + 1) * cols])
        elif fmt == D.Q4_K:
            got = O.dequantize_q4_k_row(row, cols)
            want = vals[r]
        else:
            got = O.dequantize_q6_k_row(row, cols)
            want = vals[r]
        if fmt in (D.Q4_0, D.Q8_0):
            assert np.array_equal(np.asarray(got, np.float32), np.asarray(want, np.float32))
        else:  # the quantization error of a K-quant on N(0, 1) values
            assert np.abs(np.asarray(got) - want).max() < (0.25 if fmt == D.Q4_K else 0.08)


def test_synthetic_qwen35_has_what_the_loader_reads(tmp_path):
    cfg = M.config_tiny(drafter=True)
    path = str(tmp_path / "tiny.gguf")
    G.write_synthetic_qwen35(path, cfg, seed=3)
    g = G.Gguf(path)
    assert g.str("general.architecture") == "qwen35"
    assert g.u32("qwen35.block_count") == cfg.layers + 1
    assert g.u32("qwen35.nextn_predict_layers") == 1
    assert g.u32("qwen35.embedding_length") == cfg.hidden
    assert g.u32("qwen35.ssm.inner_size") == cfg.v_heads * cfg.state_dim
    assert g.f32("qwen35.rope.freq_base") == np.float32(cfg.rope_theta)
    flags = [v.value for v in g.array("qwen35.attention.recurrent_layers")]
    assert flags == [True, True, True, False, False]
    assert g.info("token_embd.weight").dims == (cfg.hidden, cfg.vocab)
    assert g.info("output.weight").dtype == G.Q6_K
    assert g.info("blk.0.ffn_down.weight").dims == (cfg.intermediate, cfg.hidden)
    assert g.info("blk.0.ffn_down.weight").dtype == G.Q4_K
    kd, vd = cfg.k_heads * cfg.state_dim, cfg.v_heads * cfg.state_dim
    assert g.info("blk.0.attn_qkv.weight").dims == (cfg.hidden, 2 * kd + vd)
    assert g.info("blk.0.ssm_conv1d.weight").dims == (G.CONV_KERNEL, 2 * kd + vd)
    assert g.info("blk.3.attn_q.weight").dims == (cfg.hidden, 2 * cfg.heads * cfg.head_dim)
    assert g.info("blk.4.nextn.eh_proj.weight").dims == (2 * cfg.hidden, cfg.hidden)
    for name in g.tensors():
        g.bytes(name)  # every tensor lies within the file
    a = g.f32s("blk.0.ssm_a")
    assert a.shape == (cfg.v_heads,) and (a < 0).all()


@pytest.mark.gpu
def test_matrices_from_a_file_multiply_as_on_the_cpu(tmp_path):
    """Q4_K and Q6_K matrices read from a GGUF file, uploaded as they are,
    against the oracle's products of the same blocks (gpu/cpu.rs:110-149)."""
    cfg = M.config_tiny(drafter=False)
    path = str(tmp_path / "tiny.gguf")
    G.write_synthetic_qwen35(path, cfg, seed=5)
    g = G.Gguf(path)
    gpu = D.Hip(0)
    x = O.Rng(9).floats(2 * cfg.hidden)
    for name in ("blk.0.ffn_gate.weight", "output.weight"):
        t = g.matrix(name)
        w = gpu.upload(t)
        out = gpu.alloc(2 * t.rows)
        gpu.matmul(out, w, gpu.buffer(x))
        ow = O.Weight(O.Q4_K if t.fmt == D.Q4_K else O.Q6_K, t.rows, t.cols, t.quants)
        want = O.matmul(ow, x)
        got = gpu.read(out)
        err = float((np.abs(got - want) / (1 + np.abs(want))).max())
        print(f"{name}: max err {err:.2e}", flush=True)
        assert err <= 1e-4
    gpu.close()
