"""Pins the CPU oracle before anything is checked against it.

Each test is one of the reference's own known-answer tests (file:line cited),
an exhaustive or closed-form check, or a brute-force restatement in float64
numpy on small shapes, chosen so that a plausible slip in the oracle (a dropped
term, a wrong index, a transposed operand) fails one of them.
"""
import math

import numpy as np
import pytest

import oracle as O

F16_MAX = 65504.0


# ---------------------------------------------------------------- gpu/float.rs
def test_f16_round_trips_every_finite_pattern():
    # gpu/cpu.rs:511-533
    for x in [0.0, -0.0, 1.0, -2.5, 0.33325195, 65504.0, -65504.0, 1e-5, -3e-7, 2.0 ** -14]:
        b = O.to_f16(x)
        assert O.to_f16(O.from_f16(b)) == b, x
    bits = np.arange(65536, dtype=np.uint32)
    vals = np.array([O.from_f16(int(b)) for b in bits], np.float32)
    finite = (bits & 0x7C00) != 0x7C00
    back = np.array([O.to_f16(float(v)) for v in vals[finite]], np.uint32)
    assert np.array_equal(back, bits[finite])
    # closed form: numpy's IEEE half agrees on every finite pattern
    want = bits[finite].astype(np.uint16).view(np.float16).astype(np.float32)
    assert np.array_equal(vals[finite], want)


def test_f16_rounds_to_nearest_and_clamps():
    # gpu/cpu.rs:561-575
    assert O.from_f16(O.to_f16(1.0 + 2.0 ** -11)) == 1.0
    assert O.from_f16(O.to_f16(1.0 + 3.0 * 2.0 ** -11)) == 1.0 + 2.0 ** -9
    assert O.from_f16(O.to_f16(0.1)) == np.float32(0.099975586)
    assert O.from_f16(O.to_f16(1e6)) == F16_MAX
    assert O.from_f16(O.to_f16(-1e6)) == -F16_MAX
    assert O.from_f16(O.to_f16(1e-9)) == 0.0


def test_to_f16_matches_numpy_on_random_floats():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.normal(0, s, 4000) for s in (1e-6, 1e-3, 1, 1e3, 3e4)]).astype(np.float32)
    got = np.array([O.to_f16(float(v)) for v in x], np.uint16)
    want = np.clip(x, -F16_MAX, F16_MAX).astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_bf16_rounds_ties_to_even():
    assert O.to_bf16(1.0) == 0x3F80
    # 1 + 2^-8 is a tie between 0x3F80 and 0x3F81: even wins.
    assert O.to_bf16(1.0 + 2.0 ** -8) == 0x3F80
    assert O.to_bf16(1.0 + 3 * 2.0 ** -8) == 0x3F82


# ---------------------------------------------------------------- cache quantizer
def test_quantize_rounds_to_the_nearest_multiple_of_the_scale():
    # gpu/cpu.rs:536-558
    block = np.zeros(32, np.float32)
    block[:8] = [127.0, 0.5, 1.5, -2.5, 0.49, -0.51, 126.6, -0.0]
    scale, q = O.quantize(block)
    assert O.from_f16(scale) == 1.0
    assert list(q[:8]) == [127, 1, 2, -3, 0, -1, 127, 0]
    block = (np.arange(32, dtype=np.float32) - np.float32(13.3)) * np.float32(0.37)
    scale, q = O.quantize(block)
    d = O.from_f16(scale)
    assert np.all(np.abs(block - q.astype(np.float32) * np.float32(d)) <= d / 2)
    assert np.abs(q.astype(int)).max() == 127
    s, q = O.quantize(np.zeros(32))
    assert s == 0 and not q.any()
    s, q = O.quantize(np.full(32, -1e8))
    assert O.from_f16(s) == F16_MAX and np.all(q == -127)


def test_quantize_edge_blocks_follow_the_midpoint_rule():
    # the edge blocks of gpu/tests.rs:705-714, checked against exact rational
    # rounding (fractions) rather than against a restatement of the code
    from fractions import Fraction
    edges = [[127.0, 0.5, 1.5, -2.5, 126.5, -0.0, 3.5000002, -3.4999998],
             [1e6, -1e6, 65504.0, 65520.0, 0.1], [1e-3, -3e-7, 2e-4, 1e-9],
             [1e-6, 7e-7, -3e-7], [1e-9, -1e-12], [0.0],
             [0.3, 0.3 / 127.0 * 64.5, -0.3 / 127.0 * 0.5]]
    for e in edges:
        block = np.zeros(32, np.float32)
        block[:len(e)] = e
        s, q = O.quantize(block)
        amax = float(np.abs(block).max())
        assert s == O.to_f16(float(np.float32(amax) * np.float32(1.0 / 127.0)))
        d = Fraction(O.from_f16(s))
        for x, qi in zip(block, q):
            if d == 0:
                assert qi == 0
                continue
            a = Fraction(float(abs(x)))
            n = math.floor(a / d)
            if a - n * d >= d / 2:  # ties away from zero
                n += 1
            n = min(n, 127)
            assert qi == (-n if x < 0 else n), (x, qi, n)


# ---------------------------------------------------------------- Q4_0 / Q8_0
def test_q4_0_puts_the_largest_weight_at_minus_eight():
    # gpu/quant.rs:213-230
    x = np.zeros(32, np.float32)
    x[5], x[20], x[31] = -0.5, 0.25, 0.125
    s, q = O.quantize_q4_0_row(x)
    assert O.from_f16(int(s[0])) == 0.0625
    assert q[5] & 0xF == 0
    assert q[4] >> 4 == 12
    assert q[15] >> 4 == 10
    assert q[0] == 0x88
    assert np.array_equal(O.dequantize_q4_0_row(s, q), x)


def test_q8_0_round_trips_within_a_step():
    # gpu/quant.rs:197-211
    x = O.Rng(1).floats(256)
    s, q = O.quantize_q8_0_row(x)
    back = O.dequantize_q8_0_row(s, q)
    for b in range(8):
        blk = x[32 * b:32 * b + 32]
        step = np.abs(blk).max() / 127
        assert np.all(np.abs(blk - back[32 * b:32 * b + 32]) <= step * 0.51)


@pytest.mark.parametrize("cols", [32, 1024, 5120])
def test_dots_match_dequantized(cols):
    # gpu/quant.rs:232-257, plus a float64 bound
    w = O.Rng(2).floats(cols)
    x = O.Rng(3).floats(cols)
    s, q = O.quantize_q8_0_row(w)
    want = float(np.dot(O.dequantize_q8_0_row(s, q).astype(np.float64), x))
    assert abs(O.dot_q8_0(s, q, x) - want) < 1e-4 * cols
    s, q = O.quantize_q4_0_row(w)
    want = float(np.dot(O.dequantize_q4_0_row(s, q).astype(np.float64), x))
    assert abs(O.dot_q4_0(s, q, x) - want) < 1e-4 * cols


def test_rng_reproduces_the_reference_lcg():
    # gpu/tests.rs:45-54, computed with Python integers
    s, vals = 7, []
    for _ in range(5):
        s = (s * 6364136223846793005 + 1442695040888963407) % (1 << 64)
        vals.append(np.float32((s >> 40) / float(1 << 24) * 2.0 - 1.0))
    assert np.array_equal(O.Rng(7).floats(5), np.array(vals, np.float32))


# ---------------------------------------------------------------- file blocks
def test_q4_1_adds_the_minimum():
    # inference/quants.rs:222-233
    block = bytearray()
    block += O.to_f16(0.5).to_bytes(2, "little")
    block += O.to_f16(-2.0).to_bytes(2, "little")
    block += bytes((j | (15 - j) << 4) for j in range(16))
    out = O.dequantize_q4_1_file(np.frombuffer(bytes(block), np.uint8), 32)
    for j in range(16):
        assert out[j] == j * 0.5 - 2.0
        assert out[j + 16] == (15 - j) * 0.5 - 2.0


def test_q6_k_places_bits_and_scales_as_llama_cpp_does():
    # inference/quants.rs:235-275
    block = np.zeros(210, np.uint8)
    block[37] = 0b1010
    block[128 + 5] = 0b1100
    block[128 + 64 + 2] = 3
    block[208:210] = np.frombuffer(O.to_f16(0.25).to_bytes(2, "little"), np.uint8)
    out = O.dequantize_q6_k_row(block, 256)
    for i, v in enumerate(out):
        want = 19.5 if i == 37 else (0.25 * 3.0 * -32.0 if 32 <= i < 48 else 0.0)
        assert v == want, i
    block = np.zeros(210, np.uint8)
    block[64 + 36] = 0b0111_0000
    block[128 + 32 + 4] = 0b0100_0000
    block[128 + 64 + 14] = 0xFF
    block[208:210] = np.frombuffer(O.to_f16(1.0).to_bytes(2, "little"), np.uint8)
    out = O.dequantize_q6_k_row(block, 256)
    for i, v in enumerate(out):
        want = -(7.0 + 16.0 - 32.0) if i == 228 else (32.0 if 224 <= i < 240 else 0.0)
        assert v == want, i


def test_q6_k_quantizer_round_trips_and_dot_matches_dequantized():
    x = (O.Rng(31).floats(4 * 256) * 0.05).astype(np.float32)
    blocks = O.quantize_q6_k_row(x)
    back = O.dequantize_q6_k_row(blocks, x.size)
    errs = []
    for s in range(x.size // 16):
        blk = blocks[210 * (s // 16):210 * (s // 16 + 1)]
        d = O.from_f16(int(blk[208]) | int(blk[209]) << 8)
        ds = abs(d * int(np.int8(blk[192 + s % 16])))
        g = x[16 * s:16 * s + 16]
        # the group's scale covers its largest magnitude, so every weight is
        # within a step (half a step but where +32 is clipped to +31)
        assert ds >= np.abs(g).max() / 32 - 1e-9
        err = np.abs(g - back[16 * s:16 * s + 16])
        assert err.max() <= ds + 1e-7
        errs.append(err / ds)
    assert np.mean(errs) < 0.3  # rounding to nearest: a quarter step on average
    xa = O.Rng(32).floats(x.size)
    want = float(np.dot(back.astype(np.float64), xa))
    assert abs(O.dot_q6_k(blocks, xa) - want) < 1e-5 * x.size


# ---------------------------------------------------------------- Q4_K
def _q4_k_block(d, dmin, sc, mins, qs):
    """A block_q4_K built by hand from the ggml packing rules."""
    s = [0] * 12
    for j in range(8):
        if j < 4:
            s[j] = sc[j]
            s[j + 4] = mins[j]
        else:
            s[j + 4] = (sc[j] & 0xF) | ((mins[j] & 0xF) << 4)
            s[j - 4] |= (sc[j] >> 4) << 6
            s[j] |= (mins[j] >> 4) << 6
    blk = O.to_f16(d).to_bytes(2, "little") + O.to_f16(dmin).to_bytes(2, "little") + bytes(s) + bytes(qs)
    return np.frombuffer(blk, np.uint8).copy()


def test_q4_k_unpacks_six_bit_scales_and_mins_of_both_halves():
    sc = [1, 63, 5, 17, 33, 2, 63, 48]
    mins = [0, 7, 63, 1, 45, 62, 3, 16]
    qs = [0] * 128
    # sub-block j, element l: nibble j%2 of byte 32(j//2)+l; put q = (l + j) % 16
    for j in range(8):
        for l in range(32):
            qs[32 * (j // 2) + l] |= ((l + j) % 16) << (4 * (j % 2))
    blk = _q4_k_block(0.5, 0.25, sc, mins, qs)
    got = O.dequantize_q4_k_row(blk, 256)
    for j in range(8):
        for l in range(32):
            want = 0.5 * sc[j] * ((l + j) % 16) - 0.25 * mins[j]
            assert got[32 * j + l] == np.float32(want), (j, l)


def test_q4_k_single_weight_placements():
    # weight 32*5+9: sub-block 5 (high nibble of byte 64+9), scale 37 (top bits in byte 1),
    # min 40 (top bits in byte 5)
    sc = [0] * 8
    mins = [0] * 8
    sc[5], mins[5] = 37, 40
    qs = [0] * 128
    qs[64 + 9] = 0xB0
    blk = _q4_k_block(1.0, 0.5, sc, mins, qs)
    assert blk[4 + 1] >> 6 == 37 >> 4 and blk[4 + 5] >> 6 == 40 >> 4
    assert blk[4 + 9] == (37 & 0xF) | ((40 & 0xF) << 4)
    got = O.dequantize_q4_k_row(blk, 256)
    for i, v in enumerate(got):
        if i == 32 * 5 + 9:
            assert v == 37 * 11 - 20.0
        elif 160 <= i < 192:
            assert v == -20.0
        else:
            assert v == 0.0


def test_q4_k_zero_block():
    blk = O.quantize_q4_k_row(np.zeros(256, np.float32))
    assert not blk.any()
    assert not O.dequantize_q4_k_row(blk, 256).any()


def test_q4_k_quantizer_round_trips_within_a_step():
    x = (O.Rng(5).floats(8 * 256) * 0.05).astype(np.float32)
    x[:32] = np.abs(x[:32])  # a sub-block with no negative weight (min 0)
    x[32:64] = -np.abs(x[32:64]) - 0.01  # one with no positive weight
    blocks = O.quantize_q4_k_row(x)
    back = O.dequantize_q4_k_row(blocks, x.size)
    for b in range(x.size // 256):
        blk = blocks[144 * b:144 * b + 144]
        d = O.from_f16(int(blk[0]) | int(blk[1]) << 8)
        for j in range(8):
            sub = x[256 * b + 32 * j:256 * b + 32 * j + 32]
            err = np.abs(sub - back[256 * b + 32 * j:256 * b + 32 * j + 32])
            # half a step, plus the 6-bit rounding of the scale (±d/2) over 15 steps
            rng = sub.max() - min(0.0, sub.min())
            assert err.max() <= rng / 15 / 2 + 15 * d / 2 + d + 1e-6


@pytest.mark.parametrize("cols", [256, 5120])
def test_q4_k_dot_matches_dequantized(cols):
    w = (O.Rng(6).floats(cols) * 0.02).astype(np.float32)
    x = O.Rng(7).floats(cols)
    blocks = O.quantize_q4_k_row(w)
    want = float(np.dot(O.dequantize_q4_k_row(blocks, cols).astype(np.float64), x))
    assert abs(O.dot_q4_k(blocks, x) - want) < 1e-6 * cols


def test_q4_k_golden_fixture():
    """Blocks and dequantized values committed by tests/golden/make_golden.py."""
    import os
    path = os.path.join(os.path.dirname(__file__), "golden", "q4_k_q6_k.npz")
    g = np.load(path)
    assert np.array_equal(O.quantize_q4_k_row(g["x"]), g["q4_k"])
    assert np.array_equal(O.dequantize_q4_k_row(g["q4_k"], g["x"].size), g["q4_k_values"])
    assert np.array_equal(O.quantize_q6_k_row(g["x"]), g["q6_k"])
    assert np.array_equal(O.dequantize_q6_k_row(g["q6_k"], g["x"].size), g["q6_k_values"])


# ---------------------------------------------------------------- device ops
@pytest.mark.parametrize("fmt", [O.BF16, O.Q4_0, O.Q8_0, O.Q4_K, O.Q6_K])
def test_matmul_is_rows_dotted_with_tokens(fmt):
    rows, cols, n = 37, 512, 3
    vals = (O.Rng(11).floats(rows * cols) * 0.1).reshape(rows, cols)
    w = O.Weight.quantized(fmt, vals)
    x = O.Rng(12).floats(n * cols)
    got = O.matmul(w, x).reshape(n, rows)
    want = x.reshape(n, cols).astype(np.float64) @ w.dequantize().astype(np.float64).T
    assert np.allclose(got, want, rtol=0, atol=1e-5)


def test_rmsnorm_l2norm_closed_form():
    x = O.Rng(5).floats(128 * 5)
    w = O.Rng(6).floats(128)
    got = O.rmsnorm(x, w, 1e-6).reshape(5, 128)
    x64 = x.reshape(5, 128).astype(np.float64)
    want = x64 / np.sqrt((x64 ** 2).mean(1, keepdims=True) + 1e-6) * w
    assert np.allclose(got, want, rtol=1e-5, atol=1e-6)
    got = O.l2norm(x, 128, 1e-6).reshape(5, 128)
    want = x64 / np.sqrt((x64 ** 2).sum(1, keepdims=True) + 1e-6)
    assert np.allclose(got, want, rtol=1e-5, atol=1e-6)


def test_rope_is_a_complex_rotation_of_pairs_half_apart():
    n_heads, head_dim, rot, n, pos = 3, 256, 64, 2, 5
    table = O.rope_table(pos + n, rot, 1e7)
    x = O.Rng(6).floats(n * n_heads * head_dim)
    got = O.rope(x, table, pos, n_heads, head_dim, rot).reshape(n, n_heads, head_dim)
    xr = x.reshape(n, n_heads, head_dim).astype(np.float64)
    for t in range(n):
        i = np.arange(rot // 2)
        ang = (pos + t) * (1e7 ** (-(2.0 * i) / rot))
        z = (xr[t, :, :rot // 2] + 1j * xr[t, :, rot // 2:rot]) * np.exp(1j * ang)
        assert np.allclose(got[t, :, :rot // 2], z.real, atol=2e-5)
        assert np.allclose(got[t, :, rot // 2:rot], z.imag, atol=2e-5)
        assert np.array_equal(got[t, :, rot:], x.reshape(n, n_heads, head_dim)[t, :, rot:])


def test_rope_table_closed_form():
    t = O.rope_table(100, 64, 1e7).reshape(100, 32, 2)
    p = np.arange(100)[:, None]
    i = np.arange(32)[None, :]
    ang = p * 1e7 ** (-(2.0 * i) / 64)
    assert np.allclose(t[..., 0], np.cos(ang), atol=2e-5)
    assert np.allclose(t[..., 1], np.sin(ang), atol=2e-5)


@pytest.mark.parametrize("n_heads,head_dim,n_kv,n,pos", [(4, 32, 2, 3, 5), (24, 256, 4, 2, 70), (3, 96, 1, 2, 9)])
def test_attention_is_softmax_of_scaled_dots_over_the_dequantized_cache(n_heads, head_dim, n_kv, n, pos):
    rng = O.Rng(7)
    kv_dim = n_kv * head_dim
    q = rng.floats(n * n_heads * head_dim)
    kd = rng.floats((pos + n) * kv_dim)
    vd = rng.floats((pos + n) * kv_dim)
    k = O.cache_of(kd, pos * kv_dim)
    v = O.cache_of(vd, pos * kv_dim)
    got = O.attention(q, k, v, pos, n_heads, head_dim, n_kv).reshape(n, n_heads, head_dim)

    def deq(c):
        sc = np.array([O.from_f16(int(s)) for s in c.scales], np.float64)
        return (c.quants.astype(np.float64).reshape(-1, 32) * sc[:, None]).reshape(-1, n_kv, head_dim)

    K, V = deq(k), deq(v)
    qq = q.reshape(n, n_heads, head_dim).astype(np.float64)
    g = n_heads // n_kv
    for t in range(n):
        for h in range(n_heads):
            L = pos + t + 1
            s = K[:L, h // g] @ qq[t, h] / math.sqrt(head_dim)
            p = np.exp(s - s.max())
            p /= p.sum()
            assert np.allclose(got[t, h], p @ V[:L, h // g], atol=1e-5)


def test_conv_brute_force():
    qd, kd, vd = 16, 16, 48
    ch = qd + kd + vd
    for n in (1, 2, 7):
        rng = O.Rng(11 + n)
        x = rng.floats(n * ch)
        state = rng.floats(3 * ch)
        w = rng.floats(ch * 4)
        q, k, v, so = O.conv(x, state, w, qd, kd, vd)
        seq = np.concatenate([state.reshape(3, ch), x.reshape(n, ch)]).astype(np.float64)
        acc = np.stack([(seq[t:t + 4] * w.reshape(ch, 4).T).sum(0) for t in range(n)])
        y = acc / (1 + np.exp(-acc))
        got = np.concatenate([q.reshape(n, qd), k.reshape(n, kd), v.reshape(n, vd)], 1)
        assert np.allclose(got, y, atol=1e-5)
        assert np.array_equal(so.reshape(3, ch), seq[-3:].astype(np.float32))


def _delta_net_f64(q, k, v, gates, decay, state, nk, nv, d):
    n = v.size // (nv * d)
    q = q.reshape(n, nk, d).astype(np.float64)
    k = k.reshape(n, nk, d).astype(np.float64)
    v = v.reshape(n, nv, d).astype(np.float64)
    gates = gates.reshape(n, 2, nv).astype(np.float64)
    S = state.reshape(nv, d, d).astype(np.float64).copy()
    out = np.zeros((n, nv, d))
    for t in range(n):
        for h in range(nv):
            kh = h // (nv // nk)
            a = gates[t, 0, h] + decay[nv + h]
            sp = a if a > 20 else math.log1p(math.exp(a))
            g = math.exp(decay[h] * sp)
            beta = 1 / (1 + math.exp(-gates[t, 1, h]))
            S[h] *= g
            kv = S[h].T @ k[t, kh]
            S[h] += np.outer(k[t, kh], (v[t, h] - kv) * beta)
            out[t, h] = S[h].T @ q[t, kh] / math.sqrt(d)
    return out.ravel(), S.ravel()


def test_delta_net_against_float64():
    rng = O.Rng(12)
    nk, nv, d = 2, 6, 128
    for n in (1, 5):
        q, k = rng.floats(n * nk * d), rng.floats(n * nk * d)
        v = rng.floats(n * nv * d)
        gates = rng.floats(n * 2 * nv)
        decay = np.array([-abs(rng.next()) if i < nv else 4 * rng.next() for i in range(2 * nv)], np.float32)
        state = rng.floats(nv * d * d)
        out, st = O.delta_net(q, k, v, gates, decay, state, nk, nv, d)
        wo, ws = _delta_net_f64(q, k, v, gates, decay, state, nk, nv, d)
        # float32 against float64, relative to the largest magnitude (k is not
        # unit-norm here, so the state grows)
        assert np.abs(out - wo).max() <= 2e-6 * np.abs(wo).max()
        assert np.abs(st - ws).max() <= 2e-6 * np.abs(ws).max()


def test_delta_net_invariants():
    nk, nv, d = 1, 2, 128
    rng = O.Rng(3)
    state = rng.floats(nv * d * d)
    q, k, v = rng.floats(nk * d), rng.floats(nk * d), rng.floats(nv * d)
    decay = np.zeros(2 * nv, np.float32)  # a = 0: no decay
    gates = np.array([0.0] * nv + [-200.0] * nv, np.float32)  # beta = sigmoid(-200) = 0
    _, st = O.delta_net(q, k, v, gates, decay, state, nk, nv, d)
    assert np.array_equal(st, state)
    # beta = 1 and a unit key: the state then returns v for the key
    k = k / np.linalg.norm(k.astype(np.float64))
    gates = np.array([0.0] * nv + [200.0] * nv, np.float32)
    _, st = O.delta_net(q, k.astype(np.float32), v, gates, decay, state, nk, nv, d)
    S = st.reshape(nv, d, d).astype(np.float64)
    for h in range(nv):
        assert np.allclose(S[h].T @ k, v.reshape(nv, d)[h], atol=1e-4)


def test_argmax_takes_the_first_maximum():
    assert O.argmax([1.0, 3.0, 3.0, 2.0]) == 1
    assert O.argmax([-1.0]) == 0
    assert O.argmax([0.0, -0.0, 0.0]) == 0


def test_elementwise_closed_forms():
    """cpu.rs:151-155 (add), :238-242 (silu_mul: gate·σ(gate)·up, the gate
    overwritten) and :244-248 (sigmoid_mul: x·σ(gate)), against float64.  The
    operands are chosen so that exchanging them, or dropping the sigmoid,
    fails."""
    rng = O.Rng(21)
    a, b = rng.floats(4096) * np.float32(8), rng.floats(4096) * np.float32(3)
    a64, b64 = a.astype(np.float64), b.astype(np.float64)
    assert np.allclose(O.add(a, b), a64 + b64, rtol=0, atol=1e-6)
    sig = lambda v: 1 / (1 + np.exp(-v))  # noqa: E731
    got = O.silu_mul(a, b)
    want = a64 * sig(a64) * b64
    assert np.abs(got - want).max() <= 2e-6 * np.abs(want).max()
    assert np.abs(got - b64 * sig(b64) * a64).max() > 1e-2
    got = O.sigmoid_mul(a, b)
    want = a64 * sig(b64)
    assert np.abs(got - want).max() <= 2e-6 * np.abs(want).max()
    assert np.abs(got - b64 * sig(a64)).max() > 1e-2
    # exact special cases: σ(0) = 1/2, silu(0) = 0, σ(±large) saturates
    z = np.zeros(4, np.float32)
    assert np.array_equal(O.sigmoid_mul(np.full(4, 6.0, np.float32), z), np.full(4, 3.0, np.float32))
    assert np.array_equal(O.silu_mul(z, np.ones(4, np.float32)), z)
    big = np.array([100.0, -100.0], np.float32)
    assert np.array_equal(O.sigmoid_mul(np.array([5.0, 5.0], np.float32), big), np.array([5.0, 0.0], np.float32))


@pytest.mark.parametrize("n", [1, 3, 17, 70])
def test_q4_k_matmul_of_many_tokens_is_each_row_dot_bit_for_bit(n):
    """or_matmul takes Q4_K through a tiled path (nibbles converted once per
    row and tile of tokens, Σx per sub-block once per token); every element
    must carry exactly the bits of or_dot_q4_k on that row and token."""
    rows, cols = 24, 1280
    vals = (O.Rng(31).floats(rows * cols) * np.float32(0.05)).reshape(rows, cols)
    w = O.Weight.quantized(O.Q4_K, vals)
    x = O.Rng(32).floats(n * cols).reshape(n, cols)
    x[0, :7] = 0.0
    got = O.matmul(w, x).reshape(n, rows)
    q = w.quants.reshape(rows, -1)
    want = np.array([[O.dot_q4_k(q[r], x[t]) for r in range(rows)] for t in range(n)], np.float32)
    assert got.tobytes() == want.tobytes()


def test_f16_cache_stores_nearest_f16_and_attends_as_softmax_over_it():
    """The f16 KV-cache mode's oracle: stored values are numpy's float16 of
    the input (nearest, ties to even) bit for bit; attention over the cache is
    the float64 softmax of scaled dots over the f16 values."""
    rng = O.Rng(8)
    n_heads, head_dim, n_kv, n, pos = 6, 64, 2, 2, 40
    kv_dim = n_kv * head_dim
    kd = rng.floats((pos + n) * kv_dim) * np.float32(3)
    vd = rng.floats((pos + n) * kv_dim)
    kd[:3] = [65519.0, 1e-8, -2.5e-5]  # past the largest f16's halfway point, and subnormals
    k, v = O.cache_f16_of(kd), O.cache_f16_of(vd)
    assert k.read_cache(kd.size) == kd.astype(np.float16).tobytes()
    q = rng.floats(n * n_heads * head_dim)
    got = O.attention_f16(q, k, v, pos, n_heads, head_dim, n_kv).reshape(n, n_heads, head_dim)
    K = kd.astype(np.float16).astype(np.float64).reshape(-1, n_kv, head_dim)
    V = vd.astype(np.float16).astype(np.float64).reshape(-1, n_kv, head_dim)
    qq = q.reshape(n, n_heads, head_dim).astype(np.float64)
    for t in range(n):
        for h in range(n_heads):
            L = pos + t + 1
            s = K[:L, h // (n_heads // n_kv)] @ qq[t, h] / math.sqrt(head_dim)
            p = np.exp(s - s.max())
            p /= p.sum()
            assert np.allclose(got[t, h], p @ V[:L, h // (n_heads // n_kv)], atol=1e-5)
