"""The reference's `gpu::Device` trait (dwim gpu/mod.rs:176-401) over the HIP
backend's C ABI (include/dwim_hip.h), and its host `Tensor` (gpu/mod.rs:46-169).

`Hip` has one method per trait method, with the trait's argument order and
meaning; a nonzero status from the library raises `DwimError`, as the
reference's device panics on a contract violation.  Buffers, weights and
caches are handles owned by the device and freed when collected.

There is no fallback: if the built library (dwim_amd/libdwim_hip.so) is
missing, or no gfx950 GPU is present, opening the device raises.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import numpy as np

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libdwim_hip.so")

BF16, Q4_0, Q8_0, Q4_K, Q6_K = 0, 1, 2, 3, 4
FORMAT_NAMES = {BF16: "bf16", Q4_0: "q4_0", Q8_0: "q8_0", Q4_K: "q4_k", Q6_K: "q6_k"}
CACHE_BLOCK = 32
CONV_KERNEL = 4


class DwimError(RuntimeError):
    pass


_f32p = ctypes.POINTER(ctypes.c_float)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_i8p = ctypes.POINTER(ctypes.c_int8)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_vp = ctypes.c_void_p
_sz = ctypes.c_size_t
_int = ctypes.c_int

# every exported symbol of include/dwim_hip.h, with its ctypes signature
SIGNATURES = {
    "dwim_last_error": (ctypes.c_char_p, []),
    "dwim_open": (_int, [_int, ctypes.POINTER(_vp)]),
    "dwim_close": (None, [_vp]),
    "dwim_name": (_int, [_vp, ctypes.c_char_p, _sz]),
    "dwim_memory": (_int, [_vp, ctypes.POINTER(ctypes.c_uint64)]),
    "dwim_batch": (_sz, [_vp]),
    "dwim_sync": (_int, [_vp]),
    "dwim_stream": (_vp, [_vp]),
    "dwim_upload": (_int, [_vp, _int, _sz, _sz, _vp, _u16p, ctypes.POINTER(_vp)]),
    "dwim_free_weight": (None, [_vp]),
    "dwim_alloc": (_int, [_vp, _sz, ctypes.POINTER(_vp)]),
    "dwim_free_buffer": (None, [_vp]),
    "dwim_alloc_cache": (_int, [_vp, _sz, ctypes.POINTER(_vp)]),
    "dwim_alloc_cache_f16": (_int, [_vp, _sz, ctypes.POINTER(_vp)]),
    "dwim_free_cache": (None, [_vp]),
    "dwim_resize": (_int, [_vp, _vp, _sz]),
    "dwim_len": (_sz, [_vp]),
    "dwim_read": (_int, [_vp, _vp, _f32p, _sz]),
    "dwim_write": (_int, [_vp, _vp, _f32p, _sz]),
    "dwim_copy": (_int, [_vp, _vp, _sz, _vp, _sz, _sz]),
    "dwim_store": (_int, [_vp, _vp, _sz, _vp]),
    "dwim_read_cache": (_int, [_vp, _vp, _sz, _u8p, _sz]),
    "dwim_write_cache": (_int, [_vp, _vp, _u8p, _sz]),
    "dwim_cache_bytes": (_sz, [_sz]),
    "dwim_cache_bytes_of": (_sz, [_vp, _sz]),
    "dwim_matmul": (_int, [_vp, _vp, _vp, _vp]),
    "dwim_matmul_add": (_int, [_vp, _vp, _vp, _vp, _vp]),
    "dwim_swiglu": (_int, [_vp, _vp, _vp, _vp, _vp, _vp]),
    "dwim_add": (_int, [_vp, _vp, _vp]),
    "dwim_normalize": (_int, [_vp, _vp, _vp, _vp, _sz, ctypes.c_float]),
    "dwim_rmsnorm": (_int, [_vp, _vp, _vp, ctypes.c_float]),
    "dwim_l2norm": (_int, [_vp, _vp, _sz, ctypes.c_float]),
    "dwim_rope": (_int, [_vp, _vp, _vp, _sz, _sz, _sz, _sz]),
    "dwim_attention": (_int, [_vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz]),
    "dwim_attention_noalloc": (_int, [_vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz]),
    "dwim_measure_stream": (_int, [_vp, _vp, _sz, _vp, ctypes.c_uint]),
    "dwim_silu_mul": (_int, [_vp, _vp, _vp]),
    "dwim_sigmoid_mul": (_int, [_vp, _vp, _vp]),
    "dwim_conv": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "dwim_delta_net": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz]),
    "dwim_delta_net_unit_keys": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz]),
    "dwim_conv_l2norm": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, ctypes.c_float]),
    "dwim_argmax": (_int, [_vp, _vp, _sz, _u32p]),
    "dwim_sampler_open": (_int, [_vp, ctypes.c_float, _sz, ctypes.c_float, ctypes.c_float, ctypes.c_uint64,
                                 ctypes.POINTER(_vp)]),
    "dwim_sampler_free": (None, [_vp]),
    "dwim_sampler_rng": (_int, [_vp, ctypes.POINTER(ctypes.c_uint64)]),
    "dwim_sample": (_int, [_vp, _vp, _sz, _sz, _u32p]),
    "dwim_sample_verify": (_int, [_vp, _vp, _sz, _sz, ctypes.c_uint32, _u32p, ctypes.POINTER(ctypes.c_int)]),
    "dwim_prepare": (_int, [_vp, _vp]),
    "dwim_matmul_prepared": (_int, [_vp, _vp, _vp]),
    "dwim_swiglu_prepared": (_int, [_vp, _vp, _vp, _vp]),
    "dwim_embed": (_int, [_vp, _vp, _vp, _u32p, _sz]),
    "dwim_quantize_q4_0_row": (None, [_f32p, _sz, _u16p, _u8p]),
    "dwim_quantize_q8_0_row": (None, [_f32p, _sz, _u16p, _i8p]),
    "dwim_quantize_q4_k_row": (None, [_f32p, _sz, _u8p]),
    "dwim_quantize_q6_k_row": (None, [_f32p, _sz, _u8p]),
    "dwim_quantize_block": (None, [_f32p, _u16p, _i8p]),
    "dwim_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
    "dwim_from_f16": (ctypes.c_float, [ctypes.c_uint16]),
    "dwim_synthetic_values": (None, [ctypes.c_uint64, ctypes.c_uint64, _sz, ctypes.c_float, _f32p]),
    "dwim_upload_synthetic": (_int, [_vp, _int, _sz, _sz, ctypes.c_uint64, ctypes.c_float, ctypes.POINTER(_vp)]),
}

_lib = None


def lib() -> ctypes.CDLL:
    """The built library, loaded once.  Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise DwimError(f"{LIB_PATH} is not built: run `python -m dwim_amd.build` (or __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _check(status: int):
    if status != 0:
        raise DwimError(lib().dwim_last_error().decode())


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _ptr(a: np.ndarray, t):
    return a.ctypes.data_as(t)


# ------------------------------------------------------------------ host helpers
def to_f16(x: float) -> int:
    return lib().dwim_to_f16(float(x))


def from_f16(bits: int) -> float:
    return lib().dwim_from_f16(int(bits))


def quantize_block(block) -> tuple[int, np.ndarray]:
    """The cache quantizer (gpu/quant.rs:161-180) for one block of 32."""
    b = _f32(block)
    s = np.zeros(1, np.uint16)
    q = np.zeros(32, np.int8)
    lib().dwim_quantize_block(_ptr(b, _f32p), _ptr(s, _u16p), _ptr(q, _i8p))
    return int(s[0]), q


def synthetic_values(seed: int, first: int, n: int, sigma: float) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().dwim_synthetic_values(seed, first, n, sigma, _ptr(out, _f32p))
    return out


@dataclass
class Tensor:
    """A weight matrix on the host (gpu/mod.rs:46-61): bf16 bits; Q4_0/Q8_0
    quants with their block scales apart; or Q4_K/Q6_K file blocks."""

    fmt: int
    rows: int
    cols: int
    quants: np.ndarray
    scales: np.ndarray | None = None

    @property
    def shape(self):
        return (self.rows, self.cols)

    @staticmethod
    def quantize(fmt: int, values: np.ndarray) -> "Tensor":
        """Quantizes rows of f32 weights with the library's host quantizers
        (gpu/quant.rs for Q4_0/Q8_0; the ggml K-quant layouts for Q4_K/Q6_K;
        truncation to the top half for bf16, as the reference tests build it)."""
        values = _f32(values)
        rows, cols = values.shape
        L = lib()
        if fmt == BF16:
            return Tensor(BF16, rows, cols, (values.view(np.uint32) >> 16).astype(np.uint16))
        if fmt in (Q4_0, Q8_0):
            scales = np.empty(rows * cols // 32, np.uint16)
            quants = np.empty(rows * cols // (2 if fmt == Q4_0 else 1), np.uint8 if fmt == Q4_0 else np.int8)
            qpr = cols // 2 if fmt == Q4_0 else cols
            for r in range(rows):
                row = values[r]
                fn = L.dwim_quantize_q4_0_row if fmt == Q4_0 else L.dwim_quantize_q8_0_row
                fn(_ptr(row, _f32p), cols, _ptr(scales[r * cols // 32:], _u16p),
                   _ptr(quants[r * qpr:], _u8p if fmt == Q4_0 else _i8p))
            return Tensor(fmt, rows, cols, quants, scales)
        if fmt in (Q4_K, Q6_K):
            per = 144 if fmt == Q4_K else 210
            out = np.empty(rows * cols // 256 * per, np.uint8)
            fn = L.dwim_quantize_q4_k_row if fmt == Q4_K else L.dwim_quantize_q6_k_row
            bpr = cols // 256 * per
            for r in range(rows):
                row = values[r]
                fn(_ptr(row, _f32p), cols, _ptr(out[r * bpr:], _u8p))
            return Tensor(fmt, rows, cols, out)
        raise DwimError(f"unknown format {fmt}")

    def _per_row(self):
        c = self.cols
        return {BF16: (c, None), Q4_0: (c // 2, c // 32), Q8_0: (c, c // 32),
                Q4_K: (c // 256 * 144, None), Q6_K: (c // 256 * 210, None)}[self.fmt]

    def select_rows(self, rows) -> "Tensor":
        """gpu/mod.rs:74-102: the given rows, in order, repeats allowed."""
        qpr, spr = self._per_row()
        q = self.quants.reshape(self.rows, qpr)[list(rows)].ravel()
        s = None if spr is None else self.scales.reshape(self.rows, spr)[list(rows)].ravel()
        return Tensor(self.fmt, len(rows), self.cols, q, s)

    def select_column_groups(self, width: int, groups) -> "Tensor":
        """gpu/mod.rs:104-136: columns taken in groups of `width` (whole blocks)."""
        assert self.cols % width == 0
        blk = {BF16: 1, Q4_0: 32, Q8_0: 32, Q4_K: 256, Q6_K: 256}[self.fmt]
        assert width % blk == 0, "groups must be whole blocks of the format"
        qpr, spr = self._per_row()
        qg = qpr * width // self.cols
        q = self.quants.reshape(self.rows, self.cols // width, qg)[:, list(groups)].ravel()
        s = None
        if spr is not None:
            sg = spr * width // self.cols
            s = self.scales.reshape(self.rows, self.cols // width, sg)[:, list(groups)].ravel()
        return Tensor(self.fmt, self.rows, len(groups) * width, q, s)


class Buffer:
    def __init__(self, dev: "Hip", handle: int):
        self.dev, self.h = dev, handle

    def __len__(self):
        return lib().dwim_len(self.h)

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.dwim_free_buffer(self.h)
            self.h = None


class BorrowedBuffer(Buffer):
    """a buffer another object owns (freed with it, never here)"""

    def __del__(self):
        self.h = None


class Weight:
    def __init__(self, dev: "Hip", handle: int, fmt: int, rows: int, cols: int):
        self.dev, self.h, self.fmt, self.rows, self.cols = dev, handle, fmt, rows, cols

    @property
    def shape(self):
        return (self.rows, self.cols)

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.dwim_free_weight(self.h)
            self.h = None


class Cache:
    def __init__(self, dev: "Hip", handle: int, length: int):
        self.dev, self.h, self.len = dev, handle, length
        self.f16 = False

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.dwim_free_cache(self.h)
            self.h = None


class Sampler:
    """inference/sampler.rs's Sampler on the device (dwim_sampler_*): the
    same settings, the same generator, picks from a row of device logits."""

    def __init__(self, dev: "Hip", temperature: float, top_k: int, top_p: float, min_p: float, seed: int):
        self.dev = dev
        h = _vp()
        _check(lib().dwim_sampler_open(dev.h, temperature, top_k, top_p, min_p, seed, ctypes.byref(h)))
        self.h = h.value

    @property
    def rng(self) -> int:
        """the generator's state"""
        s = ctypes.c_uint64()
        _check(lib().dwim_sampler_rng(self.h, ctypes.byref(s)))
        return int(s.value)

    def sample(self, logits: Buffer, row: int = 0, vocab: int | None = None) -> int:
        """Sampler::sample of row `row` of logits ([rows][vocab])"""
        vocab = len(logits) if vocab is None else vocab
        t = ctypes.c_uint32()
        _check(lib().dwim_sample(self.h, logits.h, row, vocab, ctypes.byref(t)))
        return int(t.value)

    def verify(self, logits: Buffer, draft: int, row: int = 0, vocab: int | None = None):
        """Sampler::verify: (token, accepted)"""
        vocab = len(logits) if vocab is None else vocab
        t, a = ctypes.c_uint32(), ctypes.c_int()
        _check(lib().dwim_sample_verify(self.h, logits.h, row, vocab, draft, ctypes.byref(t), ctypes.byref(a)))
        return int(t.value), bool(a.value)

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.dwim_sampler_free(self.h)
            self.h = None


class Hip:
    """gpu::Device on an MI355X."""

    def __init__(self, index: int = 0):
        L = lib()
        h = _vp()
        _check(L.dwim_open(index, ctypes.byref(h)))
        self.h = h.value
        self.L = L

    def close(self):
        if self.h:
            self.L.dwim_close(self.h)
            self.h = None

    # ---- gpu/mod.rs:188-204
    def name(self) -> str:
        buf = ctypes.create_string_buffer(256)
        _check(self.L.dwim_name(self.h, buf, 256))
        return buf.value.decode()

    def memory(self) -> int:
        v = ctypes.c_uint64()
        _check(self.L.dwim_memory(self.h, ctypes.byref(v)))
        return v.value

    def batch(self) -> int:
        return self.L.dwim_batch(self.h)

    def sync(self):
        _check(self.L.dwim_sync(self.h))

    def stream(self) -> int:
        return self.L.dwim_stream(self.h)

    # ---- memory
    def upload(self, t: Tensor) -> Weight:
        h = _vp()
        q = np.ascontiguousarray(t.quants)
        s = None if t.scales is None else np.ascontiguousarray(t.scales, np.uint16)
        _check(self.L.dwim_upload(self.h, t.fmt, t.rows, t.cols, q.ctypes.data,
                                  None if s is None else _ptr(s, _u16p), ctypes.byref(h)))
        return Weight(self, h.value, t.fmt, t.rows, t.cols)

    def upload_synthetic(self, fmt: int, rows: int, cols: int, seed: int, sigma: float) -> Weight:
        h = _vp()
        _check(self.L.dwim_upload_synthetic(self.h, fmt, rows, cols, seed, sigma, ctypes.byref(h)))
        return Weight(self, h.value, fmt, rows, cols)

    def alloc(self, length: int) -> Buffer:
        h = _vp()
        _check(self.L.dwim_alloc(self.h, length, ctypes.byref(h)))
        return Buffer(self, h.value)

    def alloc_cache_f16(self, length: int) -> Cache:
        """An f16 key/value cache (the f16 KV-cache mode)."""
        h = _vp()
        _check(self.L.dwim_alloc_cache_f16(self.h, length, ctypes.byref(h)))
        c = Cache(self, h.value, length)
        c.f16 = True
        return c

    def alloc_cache(self, length: int) -> Cache:
        h = _vp()
        _check(self.L.dwim_alloc_cache(self.h, length, ctypes.byref(h)))
        return Cache(self, h.value, length)

    def resize(self, buf: Buffer, length: int):
        _check(self.L.dwim_resize(self.h, buf.h, length))

    def read(self, buf: Buffer) -> np.ndarray:
        n = len(buf)
        out = np.empty(n, np.float32)
        _check(self.L.dwim_read(self.h, buf.h, _ptr(out, _f32p), n))
        return out

    def write(self, buf: Buffer, data):
        d = _f32(data)
        _check(self.L.dwim_write(self.h, buf.h, _ptr(d, _f32p), d.size))

    def buffer(self, data) -> Buffer:
        """alloc + write, as gpu/tests.rs:142-146 `buffer` does."""
        d = _f32(data)
        b = self.alloc(d.size)
        self.write(b, d)
        return b

    def copy(self, dst: Buffer, dst_offset: int, src: Buffer, src_offset: int, length: int):
        _check(self.L.dwim_copy(self.h, dst.h, dst_offset, src.h, src_offset, length))

    def store(self, cache: Cache, offset: int, src: Buffer):
        _check(self.L.dwim_store(self.h, cache.h, offset, src.h))

    def read_cache(self, cache: Cache, length: int, out_bytes: int | None = None) -> bytes:
        """The cache's first `length` activations as stored; `out_bytes` (for
        tests) sizes the output below what the cache gives, to be refused."""
        need = self.L.dwim_cache_bytes_of(cache.h, length)
        out = np.empty(max(need, 1), np.uint8)
        _check(self.L.dwim_read_cache(self.h, cache.h, length, _ptr(out, _u8p),
                                      need if out_bytes is None else out_bytes))
        return out[:need].tobytes()

    def write_cache(self, cache: Cache, data: bytes):
        a = np.frombuffer(data, np.uint8).copy()
        _check(self.L.dwim_write_cache(self.h, cache.h, _ptr(a, _u8p), a.size))

    # ---- operations
    def matmul(self, out: Buffer, w: Weight, x: Buffer):
        _check(self.L.dwim_matmul(self.h, out.h, w.h, x.h))

    def matmul_add(self, x: Buffer, w: Weight, inp: Buffer, scratch: Buffer):
        _check(self.L.dwim_matmul_add(self.h, x.h, w.h, inp.h, scratch.h))

    def swiglu(self, out: Buffer, gate: Weight, up: Weight, x: Buffer, scratch: Buffer):
        _check(self.L.dwim_swiglu(self.h, out.h, gate.h, up.h, x.h, scratch.h))

    def add(self, x: Buffer, y: Buffer):
        _check(self.L.dwim_add(self.h, x.h, y.h))

    def normalize(self, out: Buffer, x: Buffer, weight: Buffer, length: int, eps: float):
        _check(self.L.dwim_normalize(self.h, out.h, x.h, weight.h, length, eps))

    def rmsnorm(self, x: Buffer, weight: Buffer, eps: float):
        _check(self.L.dwim_rmsnorm(self.h, x.h, weight.h, eps))

    def l2norm(self, x: Buffer, dim: int, eps: float):
        _check(self.L.dwim_l2norm(self.h, x.h, dim, eps))

    def rope(self, x: Buffer, table: Buffer, pos: int, n_heads: int, head_dim: int, rot_dim: int):
        _check(self.L.dwim_rope(self.h, x.h, table.h, pos, n_heads, head_dim, rot_dim))

    def attention(self, out: Buffer, q: Buffer, k: Cache, v: Cache, pos: int, n_heads: int, head_dim: int,
                  n_kv_heads: int):
        _check(self.L.dwim_attention(self.h, out.h, q.h, k.h, v.h, pos, n_heads, head_dim, n_kv_heads))

    def attention_noalloc(self, out: Buffer, q: Buffer, k: Cache, v: Cache, pos: int, n_heads: int,
                          head_dim: int, n_kv_heads: int):
        """dwim_attention without allocating: the partial results in the
        library's fixed per-GPU scratch array (no counterpart in the reference)."""
        _check(self.L.dwim_attention_noalloc(self.h, out.h, q.h, k.h, v.h, pos, n_heads, head_dim, n_kv_heads))

    def silu_mul(self, gate: Buffer, up: Buffer):
        _check(self.L.dwim_silu_mul(self.h, gate.h, up.h))

    def sigmoid_mul(self, x: Buffer, gate: Buffer):
        _check(self.L.dwim_sigmoid_mul(self.h, x.h, gate.h))

    def conv(self, q: Buffer, k: Buffer, v: Buffer, state_out: Buffer, x: Buffer, state: Buffer, weight: Buffer):
        _check(self.L.dwim_conv(self.h, q.h, k.h, v.h, state_out.h, x.h, state.h, weight.h))

    def delta_net(self, out: Buffer, q: Buffer, k: Buffer, v: Buffer, gates: Buffer, decay: Buffer,
                  state: Buffer, n_k_heads: int, n_v_heads: int, head_dim: int):
        _check(self.L.dwim_delta_net(self.h, out.h, q.h, k.h, v.h, gates.h, decay.h, state.h,
                                     n_k_heads, n_v_heads, head_dim))

    def delta_net_unit_keys(self, out: Buffer, q: Buffer, k: Buffer, v: Buffer, gates: Buffer, decay: Buffer,
                            state: Buffer, n_k_heads: int, n_v_heads: int, head_dim: int):
        """delta_net for unit keys: from 64 tokens on, the chunked form."""
        _check(self.L.dwim_delta_net_unit_keys(self.h, out.h, q.h, k.h, v.h, gates.h, decay.h, state.h,
                                               n_k_heads, n_v_heads, head_dim))

    def conv_l2norm(self, q: Buffer, k: Buffer, v: Buffer, state_out: Buffer, x: Buffer, state: Buffer,
                    weight: Buffer, dim: int, eps: float):
        """conv, then l2norm of q and k in rows of `dim`, in one launch."""
        _check(self.L.dwim_conv_l2norm(self.h, q.h, k.h, v.h, state_out.h, x.h, state.h, weight.h, dim, eps))

    def embed(self, out: Buffer, table: Weight, tokens):
        t = np.ascontiguousarray(tokens, np.uint32)
        _check(self.L.dwim_embed(self.h, out.h, table.h, _ptr(t, _u32p), t.size))

    def prepare(self, x: Buffer):
        """One token's activations as the device's int8 planes, for
        matmul_prepared (several Q4_K matrices over one x)."""
        _check(self.L.dwim_prepare(self.h, x.h))

    def matmul_prepared(self, out: Buffer, w: Weight):
        _check(self.L.dwim_matmul_prepared(self.h, out.h, w.h))

    def swiglu_prepared(self, out: Buffer, gate: Weight, up: Weight):
        """out = silu(gate·x)·(up·x) for the prepared x, as the decode step's
        feed-forward pair launch."""
        _check(self.L.dwim_swiglu_prepared(self.h, out.h, gate.h, up.h))

    def argmax(self, logits: Buffer, rows: int = 1) -> np.ndarray:
        out = np.empty(rows, np.uint32)
        _check(self.L.dwim_argmax(self.h, logits.h, rows, _ptr(out, _u32p)))
        return out

    def sampler(self, temperature: float, top_k: int, top_p: float, min_p: float, seed: int) -> Sampler:
        """Sampler::new on this device"""
        return Sampler(self, temperature, top_k, top_p, min_p, seed)


def _hip_del(self):
    try:
        self.close()
    except Exception:
        pass


Hip.__del__ = _hip_del
