"""The HIP device's operations against the CPU oracle, check by check as the
reference's device-parity suite has them (dwim gpu/tests.rs, the 18 checks of
`check_against_cpu!`, :7-42), on the same LCG inputs and with the same
tolerances (`close` :132-140, `close_batch` :198-211), plus the K-quant
formats, the device argmax and the synthetic-weight generator.

Every call goes through the C ABI (dwim_amd.device -> libdwim_hip.so)."""
import numpy as np
import pytest

import oracle as O
from dwim_amd import device as D

pytestmark = pytest.mark.gpu

OFMT = {D.BF16: O.BF16, D.Q4_0: O.Q4_0, D.Q8_0: O.Q8_0, D.Q4_K: O.Q4_K, D.Q6_K: O.Q6_K}


@pytest.fixture(scope="module")
def gpu():
    g = D.Hip(0)
    yield g
    g.close()


def close(a, b, tol):
    """gpu/tests.rs:132-140: |a-b| <= tol * (1 + max(|a|, |b|))."""
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    assert a.shape == b.shape
    bad = np.abs(a - b) > tol * (1 + np.maximum(np.abs(a), np.abs(b)))
    assert not bad.any(), f"element {np.argmax(bad)}: {a[bad][:4]} vs {b[bad][:4]}"


def close_batch(got, want, what):
    """gpu/tests.rs:198-211: rms <= 1e-3 typical, worst <= 1e-2 typical."""
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    typical = np.sqrt((want ** 2).mean())
    err = np.abs(got - want)
    rms = np.sqrt((err ** 2).mean())
    assert rms <= 1e-3 * typical and err.max() <= 1e-2 * typical, \
        f"{what}: rms {rms:.2e}, worst {err.max():.2e}, typical {typical:.2e}"


def to_tensor(w: O.Weight) -> D.Tensor:
    fmt = {v: k for k, v in OFMT.items()}[w.fmt]
    return D.Tensor(fmt, w.rows, w.cols, w.quants, w.scales)


def gcache(gpu, data, split):
    """gpu/tests.rs:149-158: a cache holding data, stored in two parts."""
    data = np.asarray(data, np.float32)
    c = gpu.alloc_cache(data.size)
    for off, part in ((0, data[:split]), (split, data[split:])):
        if part.size:
            gpu.store(c, off, gpu.buffer(part))
    return c


# ------------------------------------------------------------------ memory
def test_write_and_read_round_trip(gpu):
    data = O.Rng(1).floats(100_003)
    assert np.array_equal(gpu.read(gpu.buffer(data)), data)


def test_alloc_is_zeroed_and_copy_moves_ranges(gpu):
    assert not gpu.read(gpu.alloc(1000)).any()
    data = O.Rng(2).floats(50)
    dst = gpu.alloc(100)
    gpu.copy(dst, 30, gpu.buffer(data), 10, 20)
    want = np.zeros(100, np.float32)
    want[30:50] = data[10:30]
    assert np.array_equal(gpu.read(dst), want)


def test_resize_keeps_capacity(gpu):
    buf = gpu.alloc(64)
    gpu.resize(buf, 16)
    assert gpu.read(buf).size == 16
    gpu.resize(buf, 64)
    assert gpu.read(buf).size == 64
    with pytest.raises(D.DwimError, match="can't hold"):
        gpu.resize(buf, 65)


# ------------------------------------------------------------------ matmul
def test_matmul_matches_cpu(gpu):
    rng = O.Rng(4)
    for rows, cols, n in [(1, 8, 1), (200, 192, 1), (77, 1032, 3), (70_000, 8, 2)]:
        w = rng.bf16(rows, cols)
        x = rng.floats(n * cols)
        want = O.matmul(w, x)
        out = gpu.alloc(n * rows)
        gpu.matmul(out, gpu.upload(to_tensor(w)), gpu.buffer(x))
        close(gpu.read(out), want, 1e-4)


def test_bf16_batches_through_few_rows_match_cpu(gpu):
    # DeltaNet's gate projection shape (96 x 5120) and ragged batches
    rng = O.Rng(5)
    for rows, cols, n in [(96, 5120, 40), (128, 1024, 17), (3, 64, 300), (96, 5120, 4), (96, 5120, 1), (96, 5120, 7),
                          (5, 72, 3), (96, 2056, 15)]:
        w = rng.bf16(rows, cols)
        x = rng.floats(n * cols)
        want = O.matmul(w, x)
        out = gpu.alloc(n * rows)
        gpu.matmul(out, gpu.upload(to_tensor(w)), gpu.buffer(x))
        close(gpu.read(out), want, 1e-4)


BLOCK_SHAPES = [(1, 32, 1), (200, 5120, 1), (70_000, 32, 2), (77, 1056, 3), (200, 5120, 8), (64, 160, 9),
                (64, 128, 16), (100, 256, 47), (1030, 1152, 33), (300, 1152, 130), (2500, 5120, 64)]


def block_matmul_matches_cpu(gpu, quantized, shapes=BLOCK_SHAPES):
    """gpu/tests.rs:222-259"""
    for rows, cols, n in shapes:
        w = quantized(rows, cols)
        x = O.Rng(rows + n).floats(n * cols)
        want = O.matmul(w, x)
        out = gpu.alloc(n * rows)
        gpu.matmul(out, gpu.upload(to_tensor(w)), gpu.buffer(x))
        got = gpu.read(out)
        if n > 1:
            close_batch(got, want, f"{rows}x{cols} n={n}")
        else:
            close(got, want, 1e-4)


def test_q4_0_matmul_matches_cpu(gpu):
    rng = O.Rng(40)
    block_matmul_matches_cpu(gpu, rng.q4_0)


def test_q8_0_matmul_matches_cpu(gpu):
    rng = O.Rng(80)
    block_matmul_matches_cpu(gpu, rng.q8_0)


K_SHAPES = [(1, 256, 1), (200, 5120, 1), (7000, 256, 2), (77, 1280, 3), (200, 5120, 8), (64, 512, 9),
            (300, 1024, 33), (2500, 5120, 64), (96, 17408, 1), (130, 6144, 4)]


def _k_quantized(fmt, seed):
    rng = O.Rng(seed)

    def make(rows, cols):
        vals = (rng.floats(rows * cols) * 0.05).reshape(rows, cols)
        return O.Weight.quantized(fmt, vals)
    return make


def test_q4_k_matmul_matches_cpu(gpu):
    block_matmul_matches_cpu(gpu, _k_quantized(O.Q4_K, 44), K_SHAPES)


def test_q6_k_matmul_matches_cpu(gpu):
    block_matmul_matches_cpu(gpu, _k_quantized(O.Q6_K, 46), K_SHAPES)


def test_q6_k_few_tokens_match_cpu(gpu):
    # a verify batch through the head: runs of up to four tokens sharing the
    # weight loads (2, 3, 4, then 5 = 3 + 2 and 7 = 4 + 3), 8 waves a tile at 10240,
    # two tiles a workgroup up to 4 waves a tile (an odd tile count: the second
    # tile of the last workgroup past the rows)
    shapes = [(4000, 5120, 4), (4008, 5120, 3), (1000, 10240, 3), (33, 256, 2), (517, 2048, 5), (64, 4608, 7)]
    block_matmul_matches_cpu(gpu, _k_quantized(O.Q6_K, 47), shapes)


@pytest.mark.parametrize("rows,cols", [(17408, 5120), (5120, 17408)])
def test_q4_k_matvec_at_the_model_shapes(gpu, rows, cols):
    # W from seeded N(0, 0.02) weights, x N(0, 1), batch 1
    w = gpu.upload_synthetic(D.Q4_K, rows, cols, seed=1, sigma=0.02)
    x = D.synthetic_values(2, 0, cols, 1.0)
    out = gpu.alloc(rows)
    gpu.matmul(out, w, gpu.buffer(x))
    vals = np.stack([D.synthetic_values(1, r * cols, cols, 0.02) for r in range(0, rows, 97)])
    # rows 0, 97, 194, ... of the same synthetic weight, quantized on the host
    ow = O.Weight.quantized(O.Q4_K, vals)
    want = O.matmul(ow, x)
    close(gpu.read(out)[::97], want, 1e-4)


@pytest.mark.parametrize("rows,cols", [(17408, 5120), (5120, 17408)])
def test_q4_k_gemm_at_the_prefill_batch(gpu, rows, cols):
    """The batch product as the 4096-token prefill runs it (the f16 matrix-core
    GEMM, k-split for the 5120-row product), on every 61st row and all 4096
    tokens, against the oracle's dot of the same quantized rows: within the
    batch tolerance of gpu/tests.rs:198-211 and 1e-4 of (1 + |y|) everywhere."""
    n = 4096
    w = gpu.upload_synthetic(D.Q4_K, rows, cols, seed=3, sigma=0.02)
    x = D.synthetic_values(4, 0, n * cols, 1.0)
    out = gpu.alloc(n * rows)
    gpu.matmul(out, w, gpu.buffer(x))
    got = gpu.read(out).reshape(n, rows)[:, ::61]
    vals = np.stack([D.synthetic_values(3, r * cols, cols, 0.02) for r in range(0, rows, 61)])
    want = O.matmul(O.Weight.quantized(O.Q4_K, vals), x).reshape(n, -1)
    close_batch(got, want, f"{rows}x{cols} n={n}")
    close(got, want, 1e-4)


def test_q4_k_one_token_at_the_edges_of_its_activations(gpu):
    # one token runs on the int8 matrix cores with x held as 24-bit planes
    # scaled by max|x|: zeros, one outlier among tiny values, sign patterns
    rows, cols = 300, 2048
    w = _k_quantized(O.Q4_K, 45)(rows, cols)
    gw = gpu.upload(to_tensor(w))
    rng = np.random.default_rng(7)
    cases = {"zeros": np.zeros(cols, np.float32),
             "outlier": np.where(np.arange(cols) == 1000, 3e4, rng.normal(0, 1e-3, cols)).astype(np.float32),
             "tiny": (rng.normal(0, 1, cols) * 1e-30).astype(np.float32),
             "signs": np.where(np.arange(cols) % 2, 1.0, -1.0).astype(np.float32),
             "wide": (rng.normal(0, 1, cols) * 10.0 ** rng.uniform(-6, 3, cols)).astype(np.float32)}
    for name, x in cases.items():
        want = O.matmul(w, x)
        out = gpu.alloc(rows)
        gpu.matmul(out, gw, gpu.buffer(x))
        got = gpu.read(out)
        if name == "tiny":
            close(got / 1e-30, want / 1e-30, 1e-4)
        else:
            close(got, want, 1e-4)


def test_q4_k_near_constant_blocks(gpu):
    # blocks of nearly one value: d tiny next to dmin (the batch GEMM then
    # takes a larger unit than d for the block), next to ordinary ones
    rows, cols = 64, 1024
    rng = np.random.default_rng(9)
    vals = rng.normal(0, 0.05, (rows, cols)).astype(np.float32)
    vals[::3, :256] = 0.4 + rng.normal(0, 1e-7, (len(range(0, rows, 3)), 256))
    vals[1::3, 512:768] = -0.3 + rng.normal(0, 1e-6, (len(range(1, rows, 3)), 256))
    w = O.Weight.quantized(O.Q4_K, vals)
    gw = gpu.upload(to_tensor(w))
    for n in (1, 4, 40):
        x = O.Rng(90 + n).floats(n * cols)
        want = O.matmul(w, x)
        out = gpu.alloc(n * rows)
        gpu.matmul(out, gw, gpu.buffer(x))
        close(gpu.read(out), want, 1e-4)


def test_prepared_activations_serve_several_matrices(gpu):
    cols = 1536
    make = _k_quantized(O.Q4_K, 61)
    ws = [make(rows, cols) for rows in (64, 300)]
    x = O.Rng(62).floats(cols)
    gx = gpu.buffer(x)
    gws = [gpu.upload(to_tensor(w)) for w in ws]
    gpu.prepare(gx)
    for w, gw in zip(ws, gws):
        out = gpu.alloc(w.rows)
        gpu.matmul_prepared(out, gw)
        close(gpu.read(out), O.matmul(w, x), 1e-4)
    # a one-token matmul replaces the planes: matmul_prepared then refuses
    gpu.matmul(gpu.alloc(64), gws[0], gx)
    with pytest.raises(D.DwimError):
        gpu.matmul_prepared(gpu.alloc(64), gws[0])


def test_swiglu_prepared_matches_cpu_and_keeps_the_planes(gpu):
    """dwim_swiglu_prepared (the decode step's feed-forward pair launch over
    prepared activations): silu(gate·x)·(up·x) against the oracle, at the
    27B shape and a small one; the prepared planes stay, so it repeats."""
    for rows, cols, seed in ((17408, 5120, 63), (512, 1024, 64)):
        make = _k_quantized(O.Q4_K, seed)
        gate, up = make(rows, cols), make(rows, cols)
        x = O.Rng(seed + 1).floats(cols)
        want = O.silu_mul(O.matmul(gate, x), O.matmul(up, x))
        gpu.prepare(gpu.buffer(x))
        g, u = gpu.upload(to_tensor(gate)), gpu.upload(to_tensor(up))
        for _ in range(2):
            out = gpu.alloc(rows)
            gpu.swiglu_prepared(out, g, u)
            close(gpu.read(out), want, 1e-4)


def test_q4_k_swiglu_and_matmul_add_match_cpu(gpu):
    rng = O.Rng(24)
    # n >= 16 runs the f16 GEMM: SwiGLU in the up product's epilogue, the add,
    # and (few tiles: 4×1 here) the k split with its ordered reduce
    for rows, cols, n in [(256, 5120, 1), (1024, 1024, 1), (512, 1280, 3), (256, 512, 9), (1024, 5120, 40)]:
        make = _k_quantized(O.Q4_K, rows + n)
        gate, up = make(rows, cols), make(rows, cols)
        x = rng.floats(n * cols)
        want = O.silu_mul(O.matmul(gate, x), O.matmul(up, x))
        out, scratch = gpu.alloc(n * rows), gpu.alloc(n * rows)
        gpu.swiglu(out, gpu.upload(to_tensor(gate)), gpu.upload(to_tensor(up)), gpu.buffer(x), scratch)
        if n == 1:
            close(gpu.read(out), want, 1e-4)
        else:
            close_batch(gpu.read(out), want, f"swiglu {rows}x{cols} n={n}")
        w = make(cols, rows)
        inp = rng.floats(n * rows)
        res = rng.floats(n * cols)
        want = O.add(res, O.matmul(w, inp))
        out = gpu.buffer(res)
        gpu.matmul_add(out, gpu.upload(to_tensor(w)), gpu.buffer(inp), gpu.alloc(n * cols))
        if n == 1:
            close(gpu.read(out), want, 1e-4)
        else:
            close_batch(gpu.read(out) - res, want - res, f"matmul_add {cols}x{rows} n={n}")


def test_q4_k_small_batches_on_the_matrix_cores(gpu):
    # 2..15 tokens run on the int8 matrix cores in launches of up to four
    # tokens (7 = 4 + 3, 13 = 4 + 3 + 3 + 3); the 17408 columns split each
    # tile's blocks over several workgroups
    for rows, cols, ns in [(1100, 5120, (2, 3, 4, 5, 7, 13)), (300, 17408, (4, 6, 15)), (64, 256, (3,))]:
        w = _k_quantized(O.Q4_K, rows)(rows, cols)
        gw = gpu.upload(to_tensor(w))
        for n in ns:
            x = O.Rng(rows + n).floats(n * cols)
            want = O.matmul(w, x)
            out = gpu.alloc(n * rows)
            gpu.matmul(out, gw, gpu.buffer(x))
            got = gpu.read(out)
            for t in range(n):
                close(got[t * rows:(t + 1) * rows], want[t * rows:(t + 1) * rows], 1e-4)
            # and against the one-token product of each row of x
            one = gpu.alloc(rows)
            gpu.matmul(one, gw, gpu.buffer(x[(n - 1) * cols:]))
            close(got[(n - 1) * rows:], gpu.read(one), 1e-5)
    # a SwiGLU pair (two matrices a workgroup) and an add over split rows
    make = _k_quantized(O.Q4_K, 71)
    gate, up = make(1100, 5120), make(1100, 5120)
    x = O.Rng(72).floats(6 * 5120)
    want = O.silu_mul(O.matmul(gate, x), O.matmul(up, x))
    out, scratch = gpu.alloc(6 * 1100), gpu.alloc(6 * 1100)
    gpu.swiglu(out, gpu.upload(to_tensor(gate)), gpu.upload(to_tensor(up)), gpu.buffer(x), scratch)
    close(gpu.read(out), want, 1e-4)
    w = make(300, 17408)
    inp, res = O.Rng(73).floats(4 * 17408), O.Rng(74).floats(4 * 300)
    out = gpu.buffer(res)
    gpu.matmul_add(out, gpu.upload(to_tensor(w)), gpu.buffer(inp), gpu.alloc(4 * 300))
    close(gpu.read(out), O.add(res, O.matmul(w, inp)), 1e-4)


@pytest.mark.parametrize("fmt", [D.Q4_K, D.Q6_K, D.BF16])
def test_synthetic_weights_are_the_host_quantizers_bits(gpu, fmt):
    rows, cols = 333, 1024
    ws = gpu.upload_synthetic(fmt, rows, cols, seed=77, sigma=0.03)
    vals = D.synthetic_values(77, 0, rows * cols, 0.03).reshape(rows, cols)
    if fmt == D.BF16:
        b = vals.view(np.uint32)
        t = D.Tensor(D.BF16, rows, cols, ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16))
    else:
        t = D.Tensor.quantize(fmt, vals)
    wh = gpu.upload(t)
    x = gpu.buffer(O.Rng(3).floats(2 * cols))
    a, b = gpu.alloc(2 * rows), gpu.alloc(2 * rows)
    gpu.matmul(a, ws, x)
    gpu.matmul(b, wh, x)
    assert np.array_equal(gpu.read(a), gpu.read(b))


# ------------------------------------------------------------------ small ops
def test_rmsnorm_matches_cpu(gpu):
    rng = O.Rng(5)
    for dim, rows in [(128, 5), (1024, 3), (8, 1), (5120, 4)]:
        w = rng.floats(dim)
        x = rng.floats(dim * rows)
        buf = gpu.buffer(x)
        gpu.rmsnorm(buf, gpu.buffer(w), 1e-6)
        close(gpu.read(buf), O.rmsnorm(x, w, 1e-6), 1e-5)


def test_l2norm_matches_cpu(gpu):
    rng = O.Rng(15)
    for dim, rows in [(128, 5), (1024, 3), (8, 1)]:
        x = rng.floats(dim * rows)
        buf = gpu.buffer(x)
        gpu.l2norm(buf, dim, 1e-6)
        close(gpu.read(buf), O.l2norm(x, dim, 1e-6), 1e-5)


def test_rope_matches_cpu(gpu):
    rng = O.Rng(6)
    for n_heads, head_dim, rot_dim, n, pos in [(4, 16, 16, 3, 7), (3, 256, 64, 2, 5)]:
        table = rng.floats((pos + n) * rot_dim)
        x = rng.floats(n * n_heads * head_dim)
        buf = gpu.buffer(x)
        gpu.rope(buf, gpu.buffer(table), pos, n_heads, head_dim, rot_dim)
        close(gpu.read(buf), O.rope(x, table, pos, n_heads, head_dim, rot_dim), 1e-5)


ATTENTION_CASES = [
    (4, 32, 2, 3, 5, 1.0), (16, 128, 8, 2, 300, 1.0), (2, 128, 1, 1, 0, 1.0), (24, 256, 4, 3, 1000, 1.0),
    (3, 96, 1, 2, 9, 1.0), (2, 128, 1, 1, 0, 1e-3), (24, 256, 4, 3, 1000, 1e-3), (32, 128, 4, 64, 32704, 1.0),
    (24, 256, 4, 64, 470, 1.0), (24, 256, 4, 700, 470, 1.0), (24, 256, 4, 1, 5000, 1.0),
    (24, 256, 4, 1, 40000, 1.0), (16, 128, 8, 1, 3000, 1.0),
    # small batches: a block takes up to 4 tokens (some past a chunk's start, some not)
    (24, 256, 4, 4, 62, 1.0), (24, 256, 4, 9, 60, 1.0), (8, 64, 2, 5, 0, 1.0), (16, 128, 8, 15, 3001, 1.0),
    # the matrix-core decode pass (head_dim 256): 8 heads a key/value head and 4 tokens (32 query rows), one
    # head a key/value head past 6144 positions, a ragged last group of tokens
    (8, 256, 1, 4, 7000, 1.0), (8, 256, 8, 1, 9000, 1.0), (16, 256, 2, 9, 300, 1.0), (24, 256, 4, 2, 6143, 1e-3),
    # batches through the prefill kernel (head_dim 256, 16 tokens or more)
    (24, 256, 4, 33, 0, 1e-3), (4, 256, 1, 100, 5, 1.0), (24, 256, 4, 300, 1500, 1.0), (8, 256, 8, 16, 31, 1.0),
]


def test_attention_matches_cpu(gpu):
    """gpu/tests.rs:443-505"""
    rng = O.Rng(7)
    for n_heads, head_dim, n_kv, n, pos, size in ATTENTION_CASES:
        kv_dim = n_kv * head_dim
        q = rng.floats(n * n_heads * head_dim)
        kd = rng.floats((pos + n) * kv_dim) * np.float32(size)
        vd = rng.floats((pos + n) * kv_dim) * np.float32(size)
        want = O.attention(q, O.cache_of(kd, pos * kv_dim), O.cache_of(vd, pos * kv_dim), pos, n_heads,
                           head_dim, n_kv)
        out = gpu.alloc(q.size)
        gpu.attention(out, gpu.buffer(q), gcache(gpu, kd, pos * kv_dim), gcache(gpu, vd, pos * kv_dim), pos,
                      n_heads, head_dim, n_kv)
        close(gpu.read(out) / np.float32(size), want / np.float32(size), 1e-4)


def test_store_quantizes_like_cpu(gpu):
    """gpu/tests.rs:699-720: byte-exact."""
    data = O.Rng(9).floats(64 * 32)
    edges = [[127.0, 0.5, 1.5, -2.5, 126.5, -0.0, 3.5000002, -3.4999998], [1e6, -1e6, 65504.0, 65520.0, 0.1],
             [1e-3, -3e-7, 2e-4, 1e-9], [1e-6, 7e-7, -3e-7], [1e-9, -1e-12], [0.0],
             [0.3, 0.3 / 127.0 * 64.5, -0.3 / 127.0 * 0.5]]
    for i, e in enumerate(edges):
        data[32 * i:32 * i + 32] = 0
        data[32 * i:32 * i + len(e)] = e
    split = 11 * 32
    want = O.cache_of(data, split).read_cache(data.size)
    assert gpu.read_cache(gcache(gpu, data, split), data.size) == want


def test_cache_round_trips(gpu):
    """gpu/tests.rs:722-745"""
    length = 32 * 32
    data = O.Rng(10).floats(length)
    c = gcache(gpu, data, 7 * 32)
    blocks = [O.quantize(data[32 * i:32 * i + 32]) for i in range(32)]

    def as_bytes(bl):
        return b"".join(q.tobytes() for _, q in bl) + b"".join(int(s).to_bytes(2, "little") for s, _ in bl)

    assert gpu.read_cache(c, length) == as_bytes(blocks)
    assert gpu.read_cache(c, 3 * 32) == as_bytes(blocks[:3])
    written = list(blocks)
    for i in range(13):
        written[i] = (i * 3, np.array([(i * 7 + j) % 256 for j in range(32)], np.uint8).view(np.int8))
    gpu.write_cache(c, as_bytes(written[:13]))
    assert gpu.read_cache(c, length) == as_bytes(written)


def test_elementwise_match_cpu(gpu):
    rng = O.Rng(8)
    a, b = rng.floats(3001), rng.floats(3001)
    g = gpu.buffer(a)
    up = gpu.buffer(b)
    gpu.silu_mul(g, up)
    close(gpu.read(g), O.silu_mul(a, b), 1e-6)
    x = gpu.buffer(a)
    gpu.sigmoid_mul(x, up)
    close(gpu.read(x), O.sigmoid_mul(a, b), 1e-6)
    x = gpu.buffer(a)
    gpu.add(x, up)
    close(gpu.read(x), O.add(a, b), 1e-6)


def test_normalize_matches_cpu(gpu):
    """gpu/tests.rs:771-797"""
    rng = O.Rng(21)
    for dim, rows in [(128, 5), (1024, 3), (8, 1)]:
        w = rng.floats(dim)
        x = rng.floats(dim * (rows + 1))
        y = rng.floats(dim * rows)
        want = O.rmsnorm(x[:dim * rows], w, 1e-6)
        out = gpu.alloc(dim * rows)
        gpu.normalize(out, gpu.buffer(x), gpu.buffer(w), dim * rows, 1e-6)
        close(gpu.read(out), want, 1e-3)
        want = O.add(want, y)
        gpu.add(out, gpu.buffer(y))
        close(gpu.read(out), want, 1e-3)
        part = gpu.alloc(dim)
        gpu.copy(part, 0, out, dim * (rows - 1), dim)
        close(gpu.read(part), want[dim * (rows - 1):], 1e-3)


FUSED_SHAPES = [(64, 128, 16), (200, 5120, 1), (77, 1056, 3), (64, 160, 9), (301, 1152, 130), (2500, 512, 70)]


def test_swiglu_matches_cpu(gpu):
    rng = O.Rng(22)
    for rows, cols, n in FUSED_SHAPES:
        gate, up = rng.q4_0(rows, cols), rng.q4_0(rows, cols)
        x = rng.floats(n * cols)
        want = O.silu_mul(O.matmul(gate, x), O.matmul(up, x))
        out, scratch = gpu.alloc(n * rows), gpu.alloc(n * rows)
        gpu.swiglu(out, gpu.upload(to_tensor(gate)), gpu.upload(to_tensor(up)), gpu.buffer(x), scratch)
        close_batch(gpu.read(out), want, f"{rows}x{cols} n={n}")


def test_matmul_add_matches_cpu(gpu):
    rng = O.Rng(23)
    for rows, cols, n in FUSED_SHAPES:
        for w in (rng.q4_0(rows, cols), rng.q8_0(rows, cols), rng.bf16(rows, cols)):
            inp = rng.floats(n * cols)
            x = rng.floats(n * rows)
            want = O.add(x, O.matmul(w, inp))
            out = gpu.buffer(x)
            gpu.matmul_add(out, gpu.upload(to_tensor(w)), gpu.buffer(inp), gpu.alloc(n * rows))
            close_batch(gpu.read(out) - x, want - x, f"{rows}x{cols} n={n}")


def test_conv_matches_cpu(gpu):
    rng = O.Rng(11)
    qd, kd, vd = 16, 16, 48
    ch = qd + kd + vd
    for n in (1, 2, 7, 16, 37):  # 16 and 37: the 16-token blocks, whole and ragged
        x = rng.floats(n * ch)
        state = rng.floats(3 * ch)
        w = rng.floats(ch * 4)
        wq, wk, wv, ws = O.conv(x, state, w, qd, kd, vd)
        q, k, v, so = gpu.alloc(n * qd), gpu.alloc(n * kd), gpu.alloc(n * vd), gpu.alloc(3 * ch)
        gpu.conv(q, k, v, so, gpu.buffer(x), gpu.buffer(state), gpu.buffer(w))
        close(gpu.read(q), wq, 1e-5)
        close(gpu.read(k), wk, 1e-5)
        close(gpu.read(v), wv, 1e-5)
        close(gpu.read(so), ws, 1e-6)


def test_conv_l2norm_matches_cpu(gpu):
    """The model's fused conv + l2 norms (dwim_conv_l2norm): one token, a
    batch under 16 tokens (a token a block), and 16-token blocks whole and
    ragged, against the oracle's conv followed by its l2norm of q and k
    (gpu/cpu.rs:250-296, :168-175), at the 27B shape's rows of 128."""
    rng = O.Rng(15)
    qd, kd, vd, dim = 256, 256, 768, 128
    ch = qd + kd + vd
    for n in (1, 15, 16, 37, 4096):
        x = rng.floats(n * ch)
        state = rng.floats(3 * ch)
        w = rng.floats(ch * 4) * np.float32(0.5)
        wq, wk, wv, ws = O.conv(x, state, w, qd, kd, vd)
        wq, wk = O.l2norm(wq, dim, 1e-6), O.l2norm(wk, dim, 1e-6)
        q, k, v, so = gpu.alloc(n * qd), gpu.alloc(n * kd), gpu.alloc(n * vd), gpu.alloc(3 * ch)
        gpu.conv_l2norm(q, k, v, so, gpu.buffer(x), gpu.buffer(state), gpu.buffer(w), dim, 1e-6)
        print(f"conv_l2norm n={n}", flush=True)
        close(gpu.read(q), wq, 1e-5)
        close(gpu.read(k), wk, 1e-5)
        close(gpu.read(v), wv, 1e-5)
        assert np.array_equal(gpu.read(so), ws)


def test_delta_net_trait_op_keeps_the_token_loop_for_any_keys(gpu):
    """Device::delta_net takes any keys (gpu/cpu.rs:298-363): 100 tokens of
    keys that are not unit vectors, which the chunked form would not take,
    agree with the oracle."""
    rng = O.Rng(16)
    nk, nv, n = 2, 6, 100
    q, k, v, gates, decay, state = _delta_inputs(rng, n, nk, nv)
    k = k * np.float32(0.3)
    want, want_state = O.delta_net(q, k, v, gates, decay, state, nk, nv, 128)
    out, st = gpu.alloc(v.size), gpu.buffer(state)
    gpu.delta_net(out, gpu.buffer(q), gpu.buffer(k), gpu.buffer(v), gpu.buffer(gates), gpu.buffer(decay), st,
                  nk, nv, 128)
    scale = max(1.0, float(np.abs(want_state).max()))
    assert np.abs(gpu.read(st) - want_state).max() <= 1e-4 * scale
    assert np.abs(gpu.read(out) - want).max() <= 1e-4 * max(1.0, float(np.abs(want).max()))


def _delta_inputs(rng, n, nk, nv, d=128):
    q, k = rng.floats(n * nk * d), rng.floats(n * nk * d)
    v = rng.floats(n * nv * d)
    gates = rng.floats(n * 2 * nv)
    decay = np.array([-abs(rng.next()) if i < nv else 4 * rng.next() for i in range(2 * nv)], np.float32)
    state = rng.floats(nv * d * d)
    return q, k, v, gates, decay, state


def test_delta_net_matches_cpu(gpu):
    """gpu/tests.rs:882-946"""
    rng = O.Rng(12)
    nk, nv, d = 2, 6, 128
    for n in (1, 5):
        q, k, v, gates, decay, state = _delta_inputs(rng, n, nk, nv)
        want, want_state = O.delta_net(q, k, v, gates, decay, state, nk, nv, d)
        out = gpu.alloc(v.size)
        st = gpu.buffer(state)
        gpu.delta_net(out, gpu.buffer(q), gpu.buffer(k), gpu.buffer(v), gpu.buffer(gates), gpu.buffer(decay),
                      st, nk, nv, d)
        close(gpu.read(out), want, 1e-4)
        close(gpu.read(st), want_state, 1e-4)


def test_delta_net_in_chunks_matches_cpu(gpu):
    """Batches of 64 tokens and more take the chunked form of the delta rule
    (k_dn_prep + k_dn_chunks): the same outputs and final state as the
    token loop, with the conv's unit keys and queries (gpu/cpu.rs:298-363).
    63 tokens stay on the token loop; 100 ends in a partial chunk; 16/48 heads
    is the 27B shape (its blocks grouped by key head)."""
    rng = O.Rng(13)
    for nk, nv, n in ((2, 6, 63), (2, 6, 64), (2, 6, 100), (1, 4, 200), (16, 48, 300)):
        q, k, v, gates, decay, state = _delta_inputs(rng, n, nk, nv)
        for a in (q, k):
            r = a.reshape(n * nk, 128)
            r /= np.sqrt((r.astype(np.float64) ** 2).sum(1, keepdims=True)).astype(np.float32)
        want, want_state = O.delta_net(q, k, v, gates, decay, state, nk, nv, 128)
        out = gpu.alloc(v.size)
        st = gpu.buffer(state)
        gpu.delta_net_unit_keys(out, gpu.buffer(q), gpu.buffer(k), gpu.buffer(v), gpu.buffer(gates),
                                gpu.buffer(decay), st, nk, nv, 128)
        print(f"heads {nk}/{nv}, {n} tokens", flush=True)
        close(gpu.read(out), want, 1e-4)
        close(gpu.read(st), want_state, 1e-4)


def test_delta_net_chunks_agree_with_the_token_loop_at_full_size(gpu):
    """4096 tokens at the 27B shape (16/48 heads): one call takes the chunked
    form; the same tokens in calls of 63 take the token loop, the state
    carried between calls.  Outputs and final state agree to 1e-4 (the
    oracle at this size would take minutes; the two paths share no code)."""
    rng = O.Rng(14)
    nk, nv, n, step = 16, 48, 4096, 63
    q, k, v, gates, decay, state = _delta_inputs(rng, n, nk, nv)
    for a in (q, k):
        r = a.reshape(n * nk, 128)
        r /= np.sqrt((r.astype(np.float64) ** 2).sum(1, keepdims=True)).astype(np.float32)
    out = gpu.alloc(v.size)
    st = gpu.buffer(state)
    gpu.delta_net_unit_keys(out, gpu.buffer(q), gpu.buffer(k), gpu.buffer(v), gpu.buffer(gates),
                            gpu.buffer(decay), st, nk, nv, 128)
    want_state, parts = gpu.buffer(state), []
    for t0 in range(0, n, step):
        t1 = min(n, t0 + step)
        o = gpu.alloc((t1 - t0) * nv * 128)
        gpu.delta_net(o, gpu.buffer(q[t0 * nk * 128:t1 * nk * 128]), gpu.buffer(k[t0 * nk * 128:t1 * nk * 128]),
                      gpu.buffer(v[t0 * nv * 128:t1 * nv * 128]), gpu.buffer(gates[t0 * 2 * nv:t1 * 2 * nv]),
                      gpu.buffer(decay), want_state, nk, nv, 128)
        parts.append(gpu.read(o))
    close(gpu.read(out), np.concatenate(parts), 1e-4)
    close(gpu.read(st), gpu.read(want_state), 1e-4)


def test_argmax_takes_the_first_maximum(gpu):
    rng = O.Rng(30)
    rows, cols = 5, 248_320
    logits = rng.floats(rows * cols)
    logits[cols + 7] = 5.0
    logits[cols + 9] = 5.0  # a tie: the first wins
    logits[3 * cols + cols - 1] = 9.0
    got = gpu.argmax(gpu.buffer(logits), rows)
    want = [O.argmax(logits[r * cols:(r + 1) * cols]) for r in range(rows)]
    assert list(got) == want
    assert got[1] == 7 and got[3] == cols - 1
    # ties in different parts of a long row, and rows shorter than a part
    logits = np.full(cols, -1.0, np.float32)
    logits[[200_000, 100_000, 150_001]] = 3.0
    assert gpu.argmax(gpu.buffer(logits))[0] == 100_000
    for n in (1, 63, 1000, 1025):
        x = rng.floats(n)
        assert gpu.argmax(gpu.buffer(x))[0] == O.argmax(x)
