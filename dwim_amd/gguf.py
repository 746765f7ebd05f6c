"""GGUF files: the format the model ships in (dwim inference/gguf.rs,
model/gguf.rs), read through a memory map so that weights go from the page
cache to the device without a copy of the whole file.

    "GGUF" | version 3 (u32) | tensor count (u64) | key count (u64)
    keys: name | type (u32) | value
    tensors: name | dimension count (u32) | dimensions (u64 each, innermost
             first) | type (u32) | offset (u64) from the data start
    padding to the alignment (general.alignment, default 32) | tensor data

Strings are a u64 length and the bytes.  Beyond the reference, Q4_K (type
12) matrices are taken as they are, and so is Q6_K (14), which the reference
requantizes to Q8_0 (inference/gguf.rs:222-228): both are formats the HIP
backend uploads directly.

`write` restates the reference's test writer (inference/gguf.rs:246-320):
offsets padded to 32 bytes, the data start aligned to 32.
`write_synthetic_qwen35` writes a random-init qwen35 model of any shape, with
the tensor names and metadata keys the reference's loader reads
(inference/qwen35/mod.rs:58-148, 378-397, 759-867) and the layout of its test
model (inference/qwen35/mod.rs:1563-1722).
"""
from __future__ import annotations

import struct
from dataclasses import dataclass

import numpy as np

from . import device as D

# tensor types: llama.cpp's numbering (inference/gguf.rs:27-33, plus Q4_K)
F32, Q4_0, Q4_1, Q8_0, Q4_K, Q6_K, BF16 = 0, 2, 3, 8, 12, 14, 30

# metadata value types (model/gguf.rs:186-208)
U8, I8, U16, I16, U32, I32, F32V, BOOL, STR, ARRAY, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32V: "<f", BOOL: "<?",
           U64: "<Q", I64: "<q", F64: "<d"}

# (weights a block, bytes a block) of each tensor type
_BLOCKS = {F32: (1, 4), BF16: (1, 2), Q4_0: (32, 18), Q4_1: (32, 20), Q8_0: (32, 34), Q4_K: (256, 144),
           Q6_K: (256, 210)}


class GgufError(Exception):
    pass


@dataclass(frozen=True)
class Value:
    """A typed metadata value; `value` is a list of Values for ARRAY."""

    kind: int
    value: object

    def as_int(self):
        return int(self.value) if self.kind in _SCALAR and self.kind not in (F32V, F64) else None

    def as_float(self):
        return float(self.value) if self.kind in _SCALAR else None


def u32(v: int) -> Value:
    return Value(U32, int(v))


def f32(v: float) -> Value:
    return Value(F32V, float(v))


def string(s: str) -> Value:
    return Value(STR, s)


def array(values: list[Value]) -> Value:
    return Value(ARRAY, list(values))


def row_bytes(dtype: int, cols: int) -> int:
    """Bytes of a row of `cols` weights (inference/gguf.rs:36-52)."""
    if dtype not in _BLOCKS:
        raise GgufError(f"tensor type {dtype} is not supported")
    per, size = _BLOCKS[dtype]
    if cols % per:
        raise GgufError(f"a row of {cols} is not whole blocks of {per}")
    return cols // per * size


def to_bf16(x: np.ndarray) -> np.ndarray:
    """f32 to bf16 bits, rounding to nearest, ties to even (gpu/float.rs:32-36)."""
    bits = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16).astype(np.uint16)


@dataclass
class Info:
    dims: tuple
    dtype: int
    offset: int

    def size(self) -> int:
        rows = int(np.prod(self.dims[1:], dtype=np.int64)) if len(self.dims) > 1 else 1
        return rows * row_bytes(self.dtype, self.dims[0])


class _Reader:
    def __init__(self, buf):
        self.buf, self.pos = buf, 0

    def take(self, n: int) -> bytes:
        if self.pos + n > len(self.buf):
            raise GgufError("the file ends inside its header")
        b = bytes(self.buf[self.pos:self.pos + n])
        self.pos += n
        return b

    def scalar(self, fmt: str):
        return struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]

    def string(self) -> str:
        return self.take(self.scalar("<Q")).decode("utf-8")

    def value(self, kind: int) -> Value:
        if kind in _SCALAR:
            return Value(kind, self.scalar(_SCALAR[kind]))
        if kind == STR:
            return Value(STR, self.string())
        if kind == ARRAY:
            inner, n = self.scalar("<I"), self.scalar("<Q")
            return Value(ARRAY, [self.value(inner) for _ in range(n)])
        raise GgufError(f"unknown metadata type {kind}")


class Gguf:
    """A GGUF file opened for reading (inference/gguf.rs:109-160)."""

    def __init__(self, path: str):
        self.map = np.memmap(path, np.uint8, mode="r")
        r = _Reader(self.map)
        if r.take(4) != b"GGUF":
            raise GgufError(f"{path}: not a GGUF file")
        version = r.scalar("<I")
        if version != 3:
            raise GgufError(f"{path}: GGUF version {version} is not supported")
        n_tensors, n_meta = r.scalar("<Q"), r.scalar("<Q")
        self.meta: dict[str, Value] = {}
        for _ in range(n_meta):
            key = r.string()
            self.meta[key] = r.value(r.scalar("<I"))
        self.infos: dict[str, Info] = {}
        for _ in range(n_tensors):
            name = r.string()
            dims = tuple(r.scalar("<Q") for _ in range(r.scalar("<I")))
            dtype, offset = r.scalar("<I"), r.scalar("<Q")
            self.infos[name] = Info(dims, dtype, offset)
        align = self.meta.get("general.alignment")
        align = align.as_int() if align is not None and align.as_int() else 32
        self.data_start = (r.pos + align - 1) // align * align

    # metadata (model/gguf.rs:57-96)
    def _need(self, key: str) -> Value:
        if key not in self.meta:
            raise GgufError(f"missing metadata '{key}'")
        return self.meta[key]

    def u32(self, key: str) -> int:
        v = self._need(key).as_int()
        if v is None:
            raise GgufError(f"metadata '{key}' is not an integer")
        if not 0 <= v < 1 << 32:
            raise GgufError(f"metadata '{key}' does not fit a u32")
        return v

    def f32(self, key: str) -> float:
        v = self._need(key).as_float()
        if v is None:
            raise GgufError(f"metadata '{key}' is not a number")
        return float(np.float32(v))

    def str(self, key: str) -> str:
        v = self._need(key)
        if v.kind != STR:
            raise GgufError(f"metadata '{key}' is not a string")
        return v.value

    def array(self, key: str) -> list[Value]:
        v = self._need(key)
        if v.kind != ARRAY:
            raise GgufError(f"metadata '{key}' is not an array")
        return v.value

    # tensors (inference/gguf.rs:162-244)
    def tensors(self):
        return sorted(self.infos)

    def info(self, name: str) -> Info:
        if name not in self.infos:
            raise GgufError(f"missing tensor '{name}'")
        return self.infos[name]

    def bytes(self, name: str) -> np.ndarray:
        info = self.info(name)
        start, size = self.data_start + info.offset, info.size()
        if start + size > len(self.map):
            raise GgufError(f"tensor '{name}' runs past the end of the file")
        return self.map[start:start + size]

    def f32s(self, name: str) -> np.ndarray:
        if self.info(name).dtype != F32:
            raise GgufError(f"tensor '{name}' is not f32")
        return np.frombuffer(self.bytes(name), np.float32).copy()

    def matrix(self, name: str) -> D.Tensor:
        """A matrix in the form the device uploads: bf16, Q4_0, Q8_0 (file
        blocks split into quants and scales, gpu/mod.rs:46-61), Q4_K and
        Q6_K blocks as they are; f32 rounded to bf16 (inference/gguf.rs:
        209-236).  Q4_1 is not taken."""
        info = self.info(name)
        if len(info.dims) != 2:
            raise GgufError(f"tensor '{name}' is not a matrix")
        cols, rows = info.dims
        b = self.bytes(name)
        if info.dtype == BF16:
            return D.Tensor(D.BF16, rows, cols, np.frombuffer(b, np.uint16).copy())
        if info.dtype == F32:
            return D.Tensor(D.BF16, rows, cols, to_bf16(np.frombuffer(b, np.float32)))
        if info.dtype in (Q4_0, Q8_0):
            per = 18 if info.dtype == Q4_0 else 34
            blocks = np.frombuffer(b, np.uint8).reshape(-1, per)
            scales = blocks[:, :2].copy().view(np.uint16).ravel()
            quants = blocks[:, 2:].copy().ravel()
            if info.dtype == Q8_0:
                quants = quants.view(np.int8)
            return D.Tensor(D.Q4_0 if info.dtype == Q4_0 else D.Q8_0, rows, cols, quants, scales)
        if info.dtype in (Q4_K, Q6_K):
            return D.Tensor(D.Q4_K if info.dtype == Q4_K else D.Q6_K, rows, cols, np.array(b, np.uint8))
        raise GgufError(f"tensor '{name}' is of type {info.dtype}, which no device takes")


def _value_bytes(v: Value) -> bytes:
    if v.kind in _SCALAR:
        return struct.pack(_SCALAR[v.kind], v.value)
    if v.kind == STR:
        s = v.value.encode("utf-8")
        return struct.pack("<Q", len(s)) + s
    if v.kind == ARRAY:
        if not v.value:
            raise GgufError("an empty array has no element type")
        return struct.pack("<IQ", v.value[0].kind, len(v.value)) + b"".join(_value_bytes(x) for x in v.value)
    raise GgufError(f"unknown metadata type {v.kind}")


def write(path: str, meta: list[tuple[str, Value]], tensors: list[tuple[str, tuple, int, bytes]]) -> None:
    """Writes a GGUF file: the metadata, and tensors given by name,
    dimensions (innermost first), type and data (inference/gguf.rs:246-320)."""
    pad = lambda n: (n + 31) // 32 * 32
    out = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(meta)))
    for key, v in meta:
        k = key.encode("utf-8")
        out += struct.pack("<Q", len(k)) + k + struct.pack("<I", v.kind) + _value_bytes(v)
    offset = 0
    for name, dims, dtype, data in tensors:
        k = name.encode("utf-8")
        out += struct.pack("<Q", len(k)) + k + struct.pack("<I", len(dims))
        out += b"".join(struct.pack("<Q", d) for d in dims) + struct.pack("<IQ", dtype, offset)
        offset += pad(len(data))
    out += bytes(pad(len(out)) - len(out))
    with open(path, "wb") as f:
        f.write(out)
        for _, _, _, data in tensors:
            data = bytes(data)
            f.write(data + bytes(pad(len(data)) - len(data)))


def _file_blocks(t: D.Tensor) -> bytes:
    """A device Tensor back in its file layout."""
    if t.fmt in (D.Q4_K, D.Q6_K, D.BF16):
        return t.quants.tobytes()
    per = t.quants.size // t.scales.size
    blocks = np.concatenate([t.scales.view(np.uint8).reshape(-1, 2), t.quants.view(np.uint8).reshape(-1, per)], 1)
    return blocks.tobytes()


CONV_KERNEL = 4  # the causal conv's width (the reference's CONV_KERNEL)


def write_synthetic_qwen35(path: str, cfg, seed: int = 42, body: int = Q4_K, head: int = Q6_K,
                           context: int = 4096) -> None:
    """A random-init qwen35 model of `cfg`'s shape (a dwim_amd.model.Qwen35Config,
    with the drafter block when cfg.drafter is set):
    every layer a DeltaNet layer but each full_attention_interval-th, the
    tensors and metadata the reference loader reads, quantized by the
    library's host quantizers into `body` (Q4_0, Q8_0 or Q4_K) and `head`
    (any of those or Q6_K).  Weights are scaled by 1/sqrt(cols) so that the
    activations stay sane through the layers."""
    rng = np.random.default_rng(seed)
    fmt = {Q4_0: D.Q4_0, Q8_0: D.Q8_0, Q4_K: D.Q4_K, Q6_K: D.Q6_K}
    tensors: list = []

    def quant(name: str, rows: int, cols: int, dtype: int):
        w = rng.standard_normal((rows, cols), np.float32) / np.float32(np.sqrt(cols))
        tensors.append((name, (cols, rows), dtype, _file_blocks(D.Tensor.quantize(fmt[dtype], w))))

    def floats(name: str, dims: tuple, scale: float, offset: float):
        v = (rng.random(int(np.prod(dims)), np.float32) * 2 - 1) * np.float32(scale) + np.float32(offset)
        tensors.append((name, dims, F32, v.astype(np.float32).tobytes()))

    h, inter, heads, kvh, hd = cfg.hidden, cfg.intermediate, cfg.heads, cfg.kv_heads, cfg.head_dim
    kd, vd = cfg.k_heads * cfg.state_dim, cfg.v_heads * cfg.state_dim
    interval = cfg.full_attention_interval
    drafter = bool(cfg.drafter)
    blocks = cfg.layers + (1 if drafter else 0)
    quant("output.weight", cfg.vocab, h, head)
    quant("token_embd.weight", cfg.vocab, h, body)
    floats("output_norm.weight", (h,), 0.1, 1.0)
    for i in range(blocks):
        p = f"blk.{i}"
        full = (i + 1) % interval == 0 or i == cfg.layers
        if i == cfg.layers:
            quant(f"{p}.nextn.eh_proj.weight", h, 2 * h, body)
            for name in ("enorm", "hnorm", "shared_head_norm"):
                floats(f"{p}.nextn.{name}.weight", (h,), 0.1, 1.0)
        if full:
            quant(f"{p}.attn_q.weight", heads * hd * 2, h, body)
            quant(f"{p}.attn_k.weight", kvh * hd, h, body)
            quant(f"{p}.attn_v.weight", kvh * hd, h, body)
            quant(f"{p}.attn_output.weight", h, heads * hd, body)
            floats(f"{p}.attn_q_norm.weight", (hd,), 0.1, 1.0)
            floats(f"{p}.attn_k_norm.weight", (hd,), 0.1, 1.0)
        else:
            quant(f"{p}.attn_qkv.weight", 2 * kd + vd, h, body)
            quant(f"{p}.attn_gate.weight", vd, h, body)
            quant(f"{p}.ssm_out.weight", h, vd, body)
            for name in ("ssm_alpha", "ssm_beta"):
                floats(f"{p}.{name}.weight", (h, cfg.v_heads), 0.05, 0.0)
            floats(f"{p}.ssm_conv1d.weight", (CONV_KERNEL, 2 * kd + vd), 0.5, 0.0)
            floats(f"{p}.ssm_a", (cfg.v_heads,), 0.5, -0.6)
            floats(f"{p}.ssm_dt.bias", (cfg.v_heads,), 2.0, 0.0)
            floats(f"{p}.ssm_norm.weight", (cfg.state_dim,), 0.1, 1.0)
        quant(f"{p}.ffn_gate.weight", inter, h, body)
        quant(f"{p}.ffn_up.weight", inter, h, body)
        quant(f"{p}.ffn_down.weight", h, inter, body)
        floats(f"{p}.attn_norm.weight", (h,), 0.1, 1.0)
        floats(f"{p}.post_attention_norm.weight", (h,), 0.1, 1.0)
    meta = [
        ("general.architecture", string("qwen35")),
        ("qwen35.block_count", u32(blocks)),
        ("qwen35.context_length", u32(context)),
        ("qwen35.embedding_length", u32(h)),
        ("qwen35.feed_forward_length", u32(inter)),
        ("qwen35.attention.head_count", u32(heads)),
        ("qwen35.attention.head_count_kv", u32(kvh)),
        ("qwen35.attention.key_length", u32(hd)),
        ("qwen35.attention.value_length", u32(hd)),
        ("qwen35.rope.dimension_count", u32(cfg.rot_dim)),
        ("qwen35.rope.freq_base", f32(cfg.rope_theta)),
        ("qwen35.attention.layer_norm_rms_epsilon", f32(cfg.eps)),
        ("qwen35.ssm.conv_kernel", u32(CONV_KERNEL)),
        ("qwen35.ssm.state_size", u32(cfg.state_dim)),
        ("qwen35.ssm.group_count", u32(cfg.k_heads)),
        ("qwen35.ssm.time_step_rank", u32(cfg.v_heads)),
        ("qwen35.ssm.inner_size", u32(vd)),
        ("qwen35.full_attention_interval", u32(interval)),
    ]
    if drafter:
        meta.append(("qwen35.nextn_predict_layers", u32(1)))
    meta.append(("qwen35.attention.recurrent_layers",
                  array([Value(BOOL, (i + 1) % interval != 0 and i < cfg.layers) for i in range(blocks)])))
    write(path, meta, tensors)
