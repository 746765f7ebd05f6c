"""The qwen35 model (dwim inference/qwen35/mod.rs) on the HIP device, through
the library's C ABI (dwim_model_*): `Model` mirrors the reference's
`LanguageModel` calls the token loop makes (forward, reset, ...)."""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, fields

import numpy as np

from . import device as D


class Qwen35Config(ctypes.Structure):
    """qwen35::Config (inference/qwen35/mod.rs:29-56); the C struct dwim_qwen35_config."""
    _fields_ = [
        ("hidden", ctypes.c_size_t), ("intermediate", ctypes.c_size_t), ("layers", ctypes.c_size_t),
        ("heads", ctypes.c_size_t), ("kv_heads", ctypes.c_size_t), ("head_dim", ctypes.c_size_t),
        ("rot_dim", ctypes.c_size_t), ("rope_theta", ctypes.c_float), ("full_attention_interval", ctypes.c_size_t),
        ("k_heads", ctypes.c_size_t), ("v_heads", ctypes.c_size_t), ("state_dim", ctypes.c_size_t),
        ("eps", ctypes.c_float), ("vocab", ctypes.c_size_t), ("drafter", ctypes.c_int),
    ]

    def as_dict(self):
        return {name: getattr(self, name) for name, _ in self._fields_}


def config_27b(drafter: bool = False) -> Qwen35Config:
    """The 27B-shape hybrid of BASELINE.json: 64 layers, 3 gated-DeltaNet to 1
    full attention, hidden 5120, SwiGLU 17408, vocab 248320, 24/4 heads of 256
    (rot 64, theta 1e7), 16/48 DeltaNet heads of 128."""
    return Qwen35Config(hidden=5120, intermediate=17408, layers=64, heads=24, kv_heads=4, head_dim=256, rot_dim=64,
                        rope_theta=1e7, full_attention_interval=4, k_heads=16, v_heads=48, state_dim=128,
                        eps=1e-6, vocab=248320, drafter=int(drafter))


def config_tiny(drafter: bool = True) -> Qwen35Config:
    """The reference's synthetic test model (inference/qwen35/mod.rs:1563-1575):
    hidden 1024, 4 layers (+ the drafter), 4/2 heads of 256, 2/8 DeltaNet heads
    of 128, vocabulary 64."""
    return Qwen35Config(hidden=1024, intermediate=1024, layers=4, heads=4, kv_heads=2, head_dim=256, rot_dim=64,
                        rope_theta=10000.0, full_attention_interval=4, k_heads=2, v_heads=8, state_dim=128,
                        eps=1e-6, vocab=64, drafter=int(drafter))


_sigs_done = False


def _declare(L):
    global _sigs_done
    if _sigs_done:
        return
    vp, sz = ctypes.c_void_p, ctypes.c_size_t
    u32p = ctypes.POINTER(ctypes.c_uint32)
    f32p = ctypes.POINTER(ctypes.c_float)
    L.dwim_model_synthetic.restype = ctypes.c_int
    L.dwim_model_synthetic.argtypes = [vp, ctypes.POINTER(Qwen35Config), ctypes.c_uint64, ctypes.c_int, ctypes.c_int,
                                       sz, ctypes.POINTER(vp)]
    L.dwim_model_free.restype = None
    L.dwim_model_free.argtypes = [vp]
    L.dwim_model_batch.restype = sz
    L.dwim_model_batch.argtypes = [vp]
    L.dwim_model_forward.restype = ctypes.c_int
    L.dwim_model_forward.argtypes = [vp, u32p, sz, sz, f32p]
    L.dwim_model_forward_greedy.restype = ctypes.c_int
    L.dwim_model_forward_greedy.argtypes = [vp, u32p, sz, sz, u32p]
    L.dwim_model_decode_greedy.restype = ctypes.c_int
    L.dwim_model_decode_greedy.argtypes = [vp, ctypes.c_uint32, sz, sz, u32p]
    L.dwim_model_reset.restype = ctypes.c_int
    L.dwim_model_reset.argtypes = [vp]
    L.dwim_model_draft.restype = ctypes.c_int
    L.dwim_model_draft.argtypes = [vp, ctypes.c_uint32, sz, sz, u32p, ctypes.POINTER(sz)]
    L.dwim_model_verify.restype = ctypes.c_int
    L.dwim_model_verify.argtypes = [vp, u32p, sz, sz, f32p, u32p]
    L.dwim_model_rewind.restype = ctypes.c_int
    L.dwim_model_rewind.argtypes = [vp, sz]
    for name in ("dwim_model_mark", "dwim_model_rewind_to_mark"):
        getattr(L, name).restype = ctypes.c_int
        getattr(L, name).argtypes = [vp]
    L.dwim_model_add_sequence.restype = ctypes.c_int
    L.dwim_model_add_sequence.argtypes = [vp, ctypes.POINTER(sz)]
    L.dwim_model_select_sequence.restype = ctypes.c_int
    L.dwim_model_select_sequence.argtypes = [vp, sz]
    L.dwim_model_save.restype = ctypes.c_int
    L.dwim_model_save.argtypes = [vp, sz, ctypes.c_void_p, sz, ctypes.POINTER(sz)]
    L.dwim_model_restore.restype = ctypes.c_int
    L.dwim_model_restore.argtypes = [vp, ctypes.c_char_p, sz, ctypes.POINTER(sz)]
    L.dwim_model_logits.restype = ctypes.c_int
    L.dwim_model_logits.argtypes = [vp, ctypes.POINTER(vp)]
    _sigs_done = True


MODEL_SIGNATURES = ["dwim_model_synthetic", "dwim_model_free", "dwim_model_batch", "dwim_model_forward",
                    "dwim_model_forward_greedy", "dwim_model_decode_greedy", "dwim_model_reset", "dwim_model_draft", "dwim_model_verify",
                    "dwim_model_rewind", "dwim_model_mark", "dwim_model_rewind_to_mark", "dwim_model_add_sequence",
                    "dwim_model_select_sequence", "dwim_model_save", "dwim_model_restore", "dwim_model_logits"]


class Model:
    """A random-initialised qwen35 model on `dev` (a device.Hip)."""

    def __init__(self, dev: "D.Hip", cfg: Qwen35Config, seed: int, body_format: int = D.Q4_K,
                 head_format: int = D.Q6_K, max_len: int = 4096):
        self.L = D.lib()
        _declare(self.L)
        self.dev, self.cfg = dev, cfg
        h = ctypes.c_void_p()
        D._check(self.L.dwim_model_synthetic(dev.h, ctypes.byref(cfg), seed, body_format, head_format, max_len,
                                             ctypes.byref(h)))
        self.h = h.value

    def batch(self) -> int:
        return self.L.dwim_model_batch(self.h)

    def forward(self, tokens, pos: int, want_logits: bool = True) -> np.ndarray | None:
        t = np.ascontiguousarray(tokens, np.uint32)
        out = np.empty(self.cfg.vocab, np.float32) if want_logits else None
        D._check(self.L.dwim_model_forward(self.h, t.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), t.size, pos,
                                           None if out is None else out.ctypes.data_as(ctypes.POINTER(ctypes.c_float))))
        return out

    def forward_greedy(self, tokens, pos: int) -> int:
        t = np.ascontiguousarray(tokens, np.uint32)
        nxt = ctypes.c_uint32()
        D._check(self.L.dwim_model_forward_greedy(self.h, t.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), t.size,
                                                  pos, ctypes.byref(nxt)))
        return nxt.value

    def decode_greedy(self, token: int, pos: int, steps: int) -> list[int]:
        """`steps` greedy steps from `token` at `pos`, the picks fed back on the device."""
        out = np.zeros(max(steps, 1), np.uint32)
        D._check(self.L.dwim_model_decode_greedy(self.h, token, pos, steps,
                                                 out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32))))
        return [int(t) for t in out[:steps]]

    def reset(self):
        D._check(self.L.dwim_model_reset(self.h))

    def draft(self, token: int, pos: int, k: int) -> list[int]:
        """LanguageModel::draft (qwen35/mod.rs:1045-1071)."""
        out = np.zeros(max(k, 1), np.uint32)
        n = ctypes.c_size_t()
        D._check(self.L.dwim_model_draft(self.h, token, pos, k, out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)),
                                         ctypes.byref(n)))
        return [int(t) for t in out[:n.value]]

    def verify(self, tokens, pos: int, want_logits: bool = True):
        """LanguageModel::verify (qwen35/mod.rs:1073-1091): the logits after
        every token ([n][vocab]) and each row's greedy pick."""
        t = np.ascontiguousarray(tokens, np.uint32)
        rows = np.empty((t.size, self.cfg.vocab), np.float32) if want_logits else None
        greedy = np.zeros(t.size, np.uint32)
        D._check(self.L.dwim_model_verify(
            self.h, t.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), t.size, pos,
            None if rows is None else rows.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
            greedy.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32))))
        return rows, [int(g) for g in greedy]

    def rewind(self, keep: int):
        D._check(self.L.dwim_model_rewind(self.h, keep))

    def logits_buffer(self) -> "D.Buffer":
        """the model's logits on the device, as its last forward or verify left
        them (a view: the buffer stays the model's)"""
        h = ctypes.c_void_p()
        D._check(self.L.dwim_model_logits(self.h, ctypes.byref(h)))
        return D.BorrowedBuffer(self.dev, h.value)

    def mark(self) -> bool:
        D._check(self.L.dwim_model_mark(self.h))
        return True

    def rewind_to_mark(self):
        D._check(self.L.dwim_model_rewind_to_mark(self.h))

    def add_sequence(self) -> int:
        i = ctypes.c_size_t()
        D._check(self.L.dwim_model_add_sequence(self.h, ctypes.byref(i)))
        return i.value

    def select_sequence(self, seq: int):
        D._check(self.L.dwim_model_select_sequence(self.h, seq))

    def save(self, length: int) -> bytes | None:
        """LanguageModel::save (qwen35/mod.rs:905-947): the state after
        `length` positions as "dwimstat" v3 bytes, or None when there is
        none to save."""
        n = ctypes.c_size_t()
        D._check(self.L.dwim_model_save(self.h, length, None, 0, ctypes.byref(n)))
        if n.value == 0:
            return None
        out = ctypes.create_string_buffer(n.value)
        D._check(self.L.dwim_model_save(self.h, length, out, n.value, ctypes.byref(n)))
        return out.raw[:n.value]

    def restore(self, state: bytes) -> int:
        """LanguageModel::restore (qwen35/mod.rs:949-1017): the positions the
        state holds; raises on another layout, version or model."""
        n = ctypes.c_size_t()
        D._check(self.L.dwim_model_restore(self.h, state, len(state), ctypes.byref(n)))
        return n.value

    def close(self):
        if getattr(self, "h", None):
            self.L.dwim_model_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
