"""Python view of the CPU oracle (``oracle/liboracle.so``).

TEST INFRASTRUCTURE ONLY: the C restatement of the reference's CPU device
(dwim ``gpu/cpu.rs``), its quantizers and its forward pass.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg import this
module, as the checker; the product (``dwim_amd``) never does.

Every function takes and returns numpy arrays; each cites the reference
function it restates in the C source (``oracle/*.c``).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")

BF16, Q4_0, Q8_0, Q4_K, Q6_K = 0, 1, 2, 3, 4

_f32p = ctypes.POINTER(ctypes.c_float)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_i8p = ctypes.POINTER(ctypes.c_int8)
_u64p = ctypes.POINTER(ctypes.c_uint64)
_sz = ctypes.c_size_t


def build() -> str:
    """Compiles the oracle with its Makefile (gcc), returning the library path."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


class _Weight(ctypes.Structure):
    _fields_ = [
        ("fmt", ctypes.c_int),
        ("rows", _sz),
        ("cols", _sz),
        ("quants", ctypes.c_void_p),
        ("scales", _u16p),
    ]


def _declare(L):
    sig = {
        "or_bf16": (ctypes.c_float, [ctypes.c_uint16]),
        "or_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
        "or_to_bf16": (ctypes.c_uint16, [ctypes.c_float]),
        "or_from_f16": (ctypes.c_float, [ctypes.c_uint16]),
        "or_rng_floats": (None, [_u64p, _f32p, _sz]),
        "or_rng_bf16": (None, [_u64p, _u16p, _sz]),
        "or_quantize": (None, [_f32p, _u16p, _i8p]),
        "or_quantize_q8_0_row": (None, [_f32p, _sz, _u16p, _i8p]),
        "or_dequantize_q8_0_row": (None, [_u16p, _i8p, _sz, _f32p]),
        "or_dot_q8_0": (ctypes.c_float, [_u16p, _i8p, _f32p, _sz]),
        "or_quantize_q4_0_row": (None, [_f32p, _sz, _u16p, _u8p]),
        "or_dequantize_q4_0_row": (None, [_u16p, _u8p, _sz, _f32p]),
        "or_dot_q4_0": (ctypes.c_float, [_u16p, _u8p, _f32p, _sz]),
        "or_dot_bf16": (ctypes.c_float, [_u16p, _f32p, _sz]),
        "or_dequantize_q4_1_file": (None, [_u8p, _sz, _f32p]),
        "or_dequantize_q6_k_file": (None, [_u8p, _sz, _f32p]),
        "or_quantize_q4_k_row": (None, [_f32p, _sz, _u8p]),
        "or_dequantize_q4_k_row": (None, [_u8p, _sz, _f32p]),
        "or_dot_q4_k": (ctypes.c_float, [_u8p, _f32p, _sz]),
        "or_quantize_q6_k_row": (None, [_f32p, _sz, _u8p]),
        "or_dot_q6_k": (ctypes.c_float, [_u8p, _f32p, _sz]),
        "or_matmul": (None, [_f32p, ctypes.POINTER(_Weight), _f32p, _sz]),
        "or_add": (None, [_f32p, _f32p, _sz]),
        "or_rmsnorm": (None, [_f32p, _sz, _f32p, _sz, ctypes.c_float]),
        "or_l2norm": (None, [_f32p, _sz, _sz, ctypes.c_float]),
        "or_rope": (None, [_f32p, _sz, _f32p, _sz, _sz, _sz, _sz]),
        "or_store": (None, [_i8p, _u16p, _sz, _f32p, _sz]),
        "or_attention": (None, [_f32p, _f32p, _sz, _i8p, _u16p, _i8p, _u16p, _sz, _sz, _sz, _sz]),
        "or_store_f16": (None, [_u16p, _sz, _f32p, _sz]),
        "or_attention_f16": (None, [_f32p, _f32p, _sz, _u16p, _u16p, _sz, _sz, _sz, _sz]),
        "or_silu_mul": (None, [_f32p, _f32p, _sz]),
        "or_sigmoid_mul": (None, [_f32p, _f32p, _sz]),
        "or_conv": (None, [_f32p, _sz, _f32p, _sz, _f32p, _sz, _f32p, _f32p, _sz, _f32p, _f32p]),
        "or_delta_net": (None, [_f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _sz, _sz, _sz, _sz]),
        "or_argmax": (ctypes.c_uint32, [_f32p, _sz]),
        "or_xorshift_next": (ctypes.c_float, [_u64p]),
        "or_sampler_init": (None, [ctypes.c_void_p, ctypes.c_float, _sz, ctypes.c_float, ctypes.c_float,
                                   ctypes.c_uint64]),
        "or_sampler_candidates": (_sz, [ctypes.c_void_p, _f32p, _sz, ctypes.POINTER(ctypes.c_uint32), _f32p, _f32p]),
        "or_sample": (ctypes.c_uint32, [ctypes.c_void_p, _f32p, _sz]),
        "or_sampler_verify": (ctypes.c_uint32, [ctypes.c_void_p, _f32p, _sz, ctypes.c_uint32,
                                                ctypes.POINTER(ctypes.c_int)]),
        "or_rope_table": (None, [_f32p, _sz, _sz, ctypes.c_float]),
        "or_threads": (ctypes.c_int, []),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def _p(a: np.ndarray, t):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(t)


def f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


# ---- gpu/float.rs ----
def to_f16(x: float) -> int:
    return lib().or_to_f16(float(x))


def from_f16(bits: int) -> float:
    return lib().or_from_f16(int(bits))


def to_bf16(x: float) -> int:
    return lib().or_to_bf16(float(x))


# ---- gpu/tests.rs:45-103 ----
class Rng:
    """The reference tests' LCG, values in [-1, 1)."""

    def __init__(self, seed: int):
        self.state = ctypes.c_uint64(seed)

    def floats(self, n: int) -> np.ndarray:
        out = np.empty(n, np.float32)
        lib().or_rng_floats(ctypes.byref(self.state), _p(out, _f32p), n)
        return out

    def next(self) -> float:
        return float(self.floats(1)[0])

    def bf16_bits(self, n: int) -> np.ndarray:
        out = np.empty(n, np.uint16)
        lib().or_rng_bf16(ctypes.byref(self.state), _p(out, _u16p), n)
        return out

    def bf16(self, rows: int, cols: int) -> "Weight":
        return Weight(BF16, rows, cols, self.bf16_bits(rows * cols))

    def q4_0(self, rows: int, cols: int) -> "Weight":
        scales = np.empty(rows * cols // 32, np.uint16)
        quants = np.empty(rows * cols // 2, np.uint8)
        for r in range(rows):
            x = self.floats(cols)
            lib().or_quantize_q4_0_row(_p(x, _f32p), cols, _p(scales[r * cols // 32:], _u16p),
                                       _p(quants[r * cols // 2:], _u8p))
        return Weight(Q4_0, rows, cols, quants, scales)

    def q8_0(self, rows: int, cols: int) -> "Weight":
        scales = np.empty(rows * cols // 32, np.uint16)
        quants = np.empty(rows * cols, np.int8)
        for r in range(rows):
            x = self.floats(cols)
            lib().or_quantize_q8_0_row(_p(x, _f32p), cols, _p(scales[r * cols // 32:], _u16p),
                                       _p(quants[r * cols:], _i8p))
        return Weight(Q8_0, rows, cols, quants, scales)


# ---- quantizers (gpu/quant.rs; Q4_K/Q6_K per the ggml block layouts) ----
def quantize(block) -> tuple[int, np.ndarray]:
    block = f32(block)
    assert block.size == 32
    s = np.zeros(1, np.uint16)
    q = np.zeros(32, np.int8)
    lib().or_quantize(_p(block, _f32p), _p(s, _u16p), _p(q, _i8p))
    return int(s[0]), q


def quantize_q4_0_row(x):
    x = f32(x)
    s = np.zeros(x.size // 32, np.uint16)
    q = np.zeros(x.size // 2, np.uint8)
    lib().or_quantize_q4_0_row(_p(x, _f32p), x.size, _p(s, _u16p), _p(q, _u8p))
    return s, q


def dequantize_q4_0_row(s, q):
    out = np.empty(q.size * 2, np.float32)
    lib().or_dequantize_q4_0_row(_p(s, _u16p), _p(q, _u8p), out.size, _p(out, _f32p))
    return out


def dot_q4_0(s, q, x):
    x = f32(x)
    return lib().or_dot_q4_0(_p(s, _u16p), _p(q, _u8p), _p(x, _f32p), x.size)


def quantize_q8_0_row(x):
    x = f32(x)
    s = np.zeros(x.size // 32, np.uint16)
    q = np.zeros(x.size, np.int8)
    lib().or_quantize_q8_0_row(_p(x, _f32p), x.size, _p(s, _u16p), _p(q, _i8p))
    return s, q


def dequantize_q8_0_row(s, q):
    out = np.empty(q.size, np.float32)
    lib().or_dequantize_q8_0_row(_p(s, _u16p), _p(q, _i8p), out.size, _p(out, _f32p))
    return out


def dot_q8_0(s, q, x):
    x = f32(x)
    return lib().or_dot_q8_0(_p(s, _u16p), _p(q, _i8p), _p(x, _f32p), x.size)


def quantize_q4_k_row(x):
    x = f32(x)
    out = np.zeros(x.size // 256 * 144, np.uint8)
    lib().or_quantize_q4_k_row(_p(x, _f32p), x.size, _p(out, _u8p))
    return out


def dequantize_q4_k_row(blocks, cols):
    out = np.empty(cols, np.float32)
    lib().or_dequantize_q4_k_row(_p(np.ascontiguousarray(blocks, np.uint8), _u8p), cols, _p(out, _f32p))
    return out


def dot_q4_k(blocks, x):
    x = f32(x)
    return lib().or_dot_q4_k(_p(np.ascontiguousarray(blocks, np.uint8), _u8p), _p(x, _f32p), x.size)


def quantize_q6_k_row(x):
    x = f32(x)
    out = np.zeros(x.size // 256 * 210, np.uint8)
    lib().or_quantize_q6_k_row(_p(x, _f32p), x.size, _p(out, _u8p))
    return out


def dequantize_q6_k_row(blocks, cols):
    out = np.empty(cols, np.float32)
    lib().or_dequantize_q6_k_file(_p(np.ascontiguousarray(blocks, np.uint8), _u8p), cols, _p(out, _f32p))
    return out


def dot_q6_k(blocks, x):
    x = f32(x)
    return lib().or_dot_q6_k(_p(np.ascontiguousarray(blocks, np.uint8), _u8p), _p(x, _f32p), x.size)


def dequantize_q4_1_file(row, cols):
    out = np.empty(cols, np.float32)
    lib().or_dequantize_q4_1_file(_p(np.ascontiguousarray(row, np.uint8), _u8p), cols, _p(out, _f32p))
    return out


class Weight:
    """A weight matrix as the oracle multiplies it: bf16 bits, Q4_0/Q8_0 with
    scales apart (gpu/mod.rs:46-61), or Q4_K/Q6_K file blocks, row-major."""

    def __init__(self, fmt, rows, cols, quants, scales=None):
        self.fmt, self.rows, self.cols = fmt, rows, cols
        self.quants = np.ascontiguousarray(quants)
        self.scales = None if scales is None else np.ascontiguousarray(scales, np.uint16)

    def _struct(self):
        return _Weight(self.fmt, self.rows, self.cols, self.quants.ctypes.data,
                       None if self.scales is None else _p(self.scales, _u16p))

    @staticmethod
    def quantized(fmt, values: np.ndarray) -> "Weight":
        rows, cols = values.shape
        values = f32(values)
        if fmt == BF16:
            bits = (values.view(np.uint32) >> 16).astype(np.uint16)
            return Weight(BF16, rows, cols, bits)
        if fmt == Q4_0:
            parts = [quantize_q4_0_row(r) for r in values]
            return Weight(Q4_0, rows, cols, np.concatenate([p[1] for p in parts]),
                          np.concatenate([p[0] for p in parts]))
        if fmt == Q8_0:
            parts = [quantize_q8_0_row(r) for r in values]
            return Weight(Q8_0, rows, cols, np.concatenate([p[1] for p in parts]),
                          np.concatenate([p[0] for p in parts]))
        if fmt == Q4_K:
            return Weight(Q4_K, rows, cols, np.concatenate([quantize_q4_k_row(r) for r in values]))
        if fmt == Q6_K:
            return Weight(Q6_K, rows, cols, np.concatenate([quantize_q6_k_row(r) for r in values]))
        raise ValueError(fmt)

    def dequantize(self) -> np.ndarray:
        r, c = self.rows, self.cols
        if self.fmt == BF16:
            return (self.quants.astype(np.uint32) << 16).view(np.float32).reshape(r, c)
        out = np.empty((r, c), np.float32)
        for i in range(r):
            if self.fmt == Q4_0:
                out[i] = dequantize_q4_0_row(self.scales[i * c // 32:(i + 1) * c // 32],
                                             self.quants[i * c // 2:(i + 1) * c // 2])
            elif self.fmt == Q8_0:
                out[i] = dequantize_q8_0_row(self.scales[i * c // 32:(i + 1) * c // 32],
                                             self.quants[i * c:(i + 1) * c])
            elif self.fmt == Q4_K:
                out[i] = dequantize_q4_k_row(self.quants[i * c // 256 * 144:(i + 1) * c // 256 * 144], c)
            else:
                out[i] = dequantize_q6_k_row(self.quants[i * c // 256 * 210:(i + 1) * c // 256 * 210], c)
        return out


# ---- gpu/cpu.rs device ops, on numpy arrays ----
def matmul(w: Weight, x) -> np.ndarray:
    x = f32(x)
    n = x.size // w.cols
    assert n * w.cols == x.size
    out = np.empty(n * w.rows, np.float32)
    st = w._struct()
    lib().or_matmul(_p(out, _f32p), ctypes.byref(st), _p(x, _f32p), n)
    return out


def add(x, y):
    x = f32(x).copy()
    lib().or_add(_p(x, _f32p), _p(f32(y), _f32p), x.size)
    return x


def rmsnorm(x, weight, eps):
    x = f32(x).copy()
    w = f32(weight)
    lib().or_rmsnorm(_p(x, _f32p), x.size, _p(w, _f32p), w.size, eps)
    return x


def l2norm(x, dim, eps):
    x = f32(x).copy()
    lib().or_l2norm(_p(x, _f32p), x.size, dim, eps)
    return x


def rope(x, table, pos, n_heads, head_dim, rot_dim):
    x = f32(x).copy()
    t = f32(table)
    lib().or_rope(_p(x, _f32p), x.size, _p(t, _f32p), pos, n_heads, head_dim, rot_dim)
    return x


class Cache:
    """gpu/cpu.rs:16-19: int8 quants and f16 block scales."""

    def __init__(self, length: int):
        assert length % 32 == 0
        self.quants = np.zeros(length, np.int8)
        self.scales = np.zeros(length // 32, np.uint16)

    def store(self, offset: int, src):
        src = f32(src)
        assert offset % 32 == 0 and src.size % 32 == 0
        lib().or_store(_p(self.quants, _i8p), _p(self.scales, _u16p), offset, _p(src, _f32p), src.size)

    def read_cache(self, length: int) -> bytes:
        """gpu/cpu.rs:89-96: quants then little-endian f16 scales."""
        return self.quants[:length].tobytes() + self.scales[:length // 32].astype("<u2").tobytes()

    def write_cache(self, data: bytes):
        length = len(data) // 34 * 32
        assert len(data) == length + length // 32 * 2
        self.quants[:length] = np.frombuffer(data[:length], np.int8)
        sc = np.frombuffer(data[length:], "<u2")
        self.scales[:sc.size] = sc


def cache_of(data, split: int) -> Cache:
    """gpu/tests.rs:149-158: a cache holding `data`, stored in two parts."""
    data = f32(data)
    c = Cache(data.size)
    for off, part in ((0, data[:split]), (split, data[split:])):
        if part.size:
            c.store(off, part)
    return c


def attention(q, k: Cache, v: Cache, pos, n_heads, head_dim, n_kv_heads):
    q = f32(q)
    n = q.size // (n_heads * head_dim)
    out = np.empty_like(q)
    lib().or_attention(_p(out, _f32p), _p(q, _f32p), n, _p(k.quants, _i8p), _p(k.scales, _u16p),
                       _p(v.quants, _i8p), _p(v.scales, _u16p), pos, n_heads, head_dim, n_kv_heads)
    return out


class CacheF16:
    """The f16 KV-cache mode: f16 values (no reference; see or_store_f16)."""

    def __init__(self, length: int):
        assert length % 32 == 0
        self.values = np.zeros(length, np.uint16)

    def store(self, offset: int, src):
        src = f32(src)
        lib().or_store_f16(_p(self.values, _u16p), offset, _p(src, _f32p), src.size)

    def read_cache(self, length: int) -> bytes:
        return self.values[:length].astype("<u2").tobytes()


def cache_f16_of(data) -> CacheF16:
    data = f32(data)
    c = CacheF16(data.size)
    c.store(0, data)
    return c


def attention_f16(q, k: CacheF16, v: CacheF16, pos, n_heads, head_dim, n_kv_heads):
    q = f32(q)
    n = q.size // (n_heads * head_dim)
    out = np.empty_like(q)
    lib().or_attention_f16(_p(out, _f32p), _p(q, _f32p), n, _p(k.values, _u16p), _p(v.values, _u16p), pos,
                           n_heads, head_dim, n_kv_heads)
    return out


def silu_mul(gate, up):
    g = f32(gate).copy()
    lib().or_silu_mul(_p(g, _f32p), _p(f32(up), _f32p), g.size)
    return g


def sigmoid_mul(x, gate):
    x = f32(x).copy()
    lib().or_sigmoid_mul(_p(x, _f32p), _p(f32(gate), _f32p), x.size)
    return x


def conv(x, state, weight, q_dim, k_dim, v_dim):
    x, state, weight = f32(x), f32(state), f32(weight)
    ch = q_dim + k_dim + v_dim
    n = x.size // ch
    q = np.empty(n * q_dim, np.float32)
    k = np.empty(n * k_dim, np.float32)
    v = np.empty(n * v_dim, np.float32)
    so = np.empty(state.size, np.float32)
    lib().or_conv(_p(q, _f32p), q_dim, _p(k, _f32p), k_dim, _p(v, _f32p), v_dim, _p(so, _f32p),
                  _p(x, _f32p), n, _p(state, _f32p), _p(weight, _f32p))
    return q, k, v, so


def delta_net(q, k, v, gates, decay, state, n_k_heads, n_v_heads, head_dim):
    q, k, v, gates, decay = f32(q), f32(k), f32(v), f32(gates), f32(decay)
    state = f32(state).copy()
    n = v.size // (n_v_heads * head_dim)
    out = np.empty_like(v)
    lib().or_delta_net(_p(out, _f32p), _p(q, _f32p), _p(k, _f32p), _p(v, _f32p), _p(gates, _f32p),
                       _p(decay, _f32p), _p(state, _f32p), n, n_k_heads, n_v_heads, head_dim)
    return out, state


def argmax(logits) -> int:
    x = f32(logits)
    return int(lib().or_argmax(_p(x, _f32p), x.size))


# ---- inference/sampler.rs ----
class _SamplerState(ctypes.Structure):
    _fields_ = [("temperature", ctypes.c_float), ("top_k", _sz), ("top_p", ctypes.c_float),
                ("min_p", ctypes.c_float), ("rng", ctypes.c_uint64)]


def xorshift_next(state: int):
    """Rng::next (sampler.rs:136-146): (the value in [0, 1), the next state)."""
    s = ctypes.c_uint64(state)
    v = lib().or_xorshift_next(ctypes.byref(s))
    return float(v), int(s.value)


class Sampler:
    """Sampler (sampler.rs:7-133): sample and verify advance the generator
    as the reference's do."""

    def __init__(self, temperature, top_k, top_p, min_p, seed):
        self._s = _SamplerState()
        lib().or_sampler_init(ctypes.byref(self._s), temperature, top_k, top_p, min_p, seed)

    @property
    def rng(self) -> int:
        return int(self._s.rng)

    def candidates(self, logits):
        """(tokens, probabilities, total) of Sampler::candidates"""
        x = f32(logits)
        tok = np.empty(max(x.size, 1), np.uint32)
        pr = np.empty(max(x.size, 1), np.float32)
        tot = ctypes.c_float()
        n = lib().or_sampler_candidates(ctypes.byref(self._s), _p(x, _f32p), x.size,
                                        tok.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), _p(pr, _f32p),
                                        ctypes.byref(tot))
        return tok[:n].copy(), pr[:n].copy(), float(tot.value)

    def sample(self, logits) -> int:
        x = f32(logits)
        return int(lib().or_sample(ctypes.byref(self._s), _p(x, _f32p), x.size))

    def verify(self, logits, draft):
        """(token, accepted) of Sampler::verify"""
        x = f32(logits)
        acc = ctypes.c_int()
        t = lib().or_sampler_verify(ctypes.byref(self._s), _p(x, _f32p), x.size, int(draft), ctypes.byref(acc))
        return int(t), bool(acc.value)


def rope_table(max_len, rot_dim, theta):
    t = np.empty(max_len * rot_dim, np.float32)
    lib().or_rope_table(_p(t, _f32p), max_len, rot_dim, theta)
    return t


def threads() -> int:
    return lib().or_threads()


# ---- the qwen35 forward pass (inference/qwen35/mod.rs), oracle/model.c ----
class Qwen35Config(ctypes.Structure):
    _fields_ = [
        ("hidden", _sz), ("intermediate", _sz), ("layers", _sz), ("heads", _sz), ("kv_heads", _sz),
        ("head_dim", _sz), ("rot_dim", _sz), ("rope_theta", ctypes.c_float), ("full_attention_interval", _sz),
        ("k_heads", _sz), ("v_heads", _sz), ("state_dim", _sz), ("eps", ctypes.c_float), ("vocab", _sz),
        ("drafter", ctypes.c_int),
    ]


def _declare_model(L):
    if getattr(L, "_model_declared", False):
        return
    vp = ctypes.c_void_p
    u32p = ctypes.POINTER(ctypes.c_uint32)
    L.or_model_synthetic.restype = vp
    L.or_model_synthetic.argtypes = [ctypes.POINTER(Qwen35Config), ctypes.c_uint64, ctypes.c_int, ctypes.c_int, _sz, _sz]
    L.or_model_free.restype = None
    L.or_model_free.argtypes = [vp]
    L.or_model_forward.restype = None
    L.or_model_forward.argtypes = [vp, u32p, _sz, _sz, _f32p]
    L.or_model_draft.restype = _sz
    L.or_model_draft.argtypes = [vp, ctypes.c_uint32, _sz, _sz, u32p]
    L.or_model_reset.restype = None
    L.or_model_reset.argtypes = [vp]
    L.or_model_zero_residual_writes.restype = None
    L.or_model_save.restype = _sz
    L.or_model_save.argtypes = [vp, _sz, ctypes.c_void_p]
    L.or_model_restore.restype = ctypes.c_int
    L.or_model_restore.argtypes = [vp, ctypes.c_char_p, _sz, ctypes.POINTER(_sz)]
    L.or_model_zero_residual_writes.argtypes = [vp]
    L.or_model_last_logits.restype = None
    L.or_model_last_logits.argtypes = [vp, _f32p]
    L.or_model_verify.restype = None
    L.or_model_verify.argtypes = [vp, u32p, _sz, _sz, _f32p]
    L.or_model_rewind.restype = None
    L.or_model_rewind.argtypes = [vp, _sz]
    L.or_model_mark.restype = None
    L.or_model_mark.argtypes = [vp]
    L.or_model_rewind_to_mark.restype = ctypes.c_int
    L.or_model_rewind_to_mark.argtypes = [vp]
    L.or_synthetic_values.restype = None
    L.or_synthetic_values.argtypes = [ctypes.c_uint64, ctypes.c_uint64, _sz, ctypes.c_float, _f32p]
    L._model_declared = True


def synthetic_values(seed, first, n, sigma):
    L = lib()
    _declare_model(L)
    out = np.empty(n, np.float32)
    L.or_synthetic_values(seed, first, n, sigma, _p(out, _f32p))
    return out


class Model:
    """The oracle's qwen35 model for the same synthetic weights as the
    product's dwim_model_synthetic (fields as dwim_qwen35_config)."""

    def __init__(self, cfg: dict, seed: int, body_fmt=Q4_K, head_fmt=Q6_K, max_len=64, batch=64):
        L = lib()
        _declare_model(L)
        self.L, self.vocab = L, cfg["vocab"]
        self.cfg = Qwen35Config(**cfg)
        self.h = L.or_model_synthetic(ctypes.byref(self.cfg), seed, body_fmt, head_fmt, max_len, batch)

    def forward(self, tokens, pos):
        t = np.ascontiguousarray(tokens, np.uint32)
        out = np.empty(self.vocab, np.float32)
        self.L.or_model_forward(self.h, t.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), t.size, pos,
                                _p(out, _f32p))
        return out

    def draft(self, token, pos, k):
        out = np.zeros(max(k, 1), np.uint32)
        n = self.L.or_model_draft(self.h, token, pos, k, out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)))
        return list(out[:n])

    def last_logits(self):
        """The logits of the last single-token head product: after draft(),
        those its last draft was picked from."""
        out = np.empty(self.vocab, np.float32)
        self.L.or_model_last_logits(self.h, _p(out, _f32p))
        return out

    def verify(self, tokens, pos):
        t = np.ascontiguousarray(tokens, np.uint32)
        assert 0 < t.size <= 9
        out = np.empty((t.size, self.vocab), np.float32)
        self.L.or_model_verify(self.h, t.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), t.size, pos,
                               _p(out, _f32p))
        return out

    def rewind(self, keep):
        self.L.or_model_rewind(self.h, keep)

    def mark(self):
        self.L.or_model_mark(self.h)

    def rewind_to_mark(self):
        if self.L.or_model_rewind_to_mark(self.h):
            raise RuntimeError("no mark to rewind to, or a batch is being verified")

    def reset(self):
        self.L.or_model_reset(self.h)

    RESTORE_ERRORS = {1: "the saved state is cut short", 2: "not a saved state",
                      3: "a saved state of another version", 4: "a saved state of another model",
                      5: "does not fit in the context"}

    def save(self, length):
        """LanguageModel::save: the dwimstat v3 bytes, or None."""
        n = self.L.or_model_save(self.h, length, None)
        if n == 0:
            return None
        out = ctypes.create_string_buffer(n)
        self.L.or_model_save(self.h, length, out)
        return out.raw

    def restore(self, state: bytes) -> int:
        n = _sz()
        err = self.L.or_model_restore(self.h, state, len(state), ctypes.byref(n))
        if err:
            raise ValueError(self.RESTORE_ERRORS[err])
        return n.value

    def zero_residual_writes(self):
        """Test hook: every ffn_down, attn_output and ssm_out becomes zero."""
        self.L.or_model_zero_residual_writes(self.h)

    def __del__(self):
        if getattr(self, "h", None):
            self.L.or_model_free(self.h)
            self.h = None
