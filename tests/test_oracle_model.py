"""Pins the oracle's qwen35 forward pass (oracle/model.c) with an independent
float64 restatement of the reference's layer order, written in numpy from
inference/qwen35/mod.rs and gpu/cpu.rs directly, on the same random-init
weights (each tensor regenerated here from its seed and name, quantized by the
oracle's pinned quantizers and dequantized in float64):

* forward_batch (qwen35/mod.rs:425-496): embed, every layer, the final norm
  and the head on the last token;
* Pass::layer (:541-655): attention mixer (q, gate, k, v products; q/k RMS
  norms; rope; the Q8 cache; causal GQA softmax; sigmoid gate; o product
  added) or linear mixer (qkv, z, ab products; causal conv of 4 taps and SiLU
  with the carried state, cpu.rs:250-296; l2 norms; the gated delta rule,
  cpu.rs:298-363; RMS norm; silu(z)·o; out product added), then the SwiGLU
  FFN silu(gate·x)·(up·x) with the down product added;
* the state carried across calls (the conv window and the delta-rule state).

A slip in the oracle's order (gate and up swapped, the two norms swapped, a
stale conv state) moves the logits far beyond the 1e-4 this allows.  A second
check zeroes every product that writes into the residual stream: the logits
must then be head·rmsnorm(embed(token)), whatever the layers compute.
"""
import math

import numpy as np
import pytest

import oracle as O

M64 = (1 << 64) - 1
TINY = dict(hidden=1024, intermediate=1024, layers=4, heads=4, kv_heads=2, head_dim=256, rot_dim=64,
            rope_theta=10000.0, full_attention_interval=4, k_heads=2, v_heads=8, state_dim=128, eps=1e-6,
            vocab=64, drafter=0)


def _splitmix(seed, i):
    z = (seed + (i + 1) * 0x9E3779B97F4A7C15) & M64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
    return z ^ (z >> 31)


def _fnv1a(s):
    h = 0xCBF29CE484222325
    for ch in s.encode():
        h = ((h ^ ch) * 0x100000001B3) & M64
    return h


class Weights:
    """The synthetic model's tensors, regenerated from (model seed, name)."""

    def __init__(self, seed):
        self.seed = seed

    def _seed(self, name):
        return _splitmix(self.seed, _fnv1a(name))

    def vec(self, name, n, sigma=0.1, offset=1.0):
        return O.synthetic_values(self._seed(name), 0, n, sigma).astype(np.float64) + offset

    def uniform(self, name, n, scale, offset):
        s = self._seed(name)
        u = np.array([(_splitmix(s, i) >> 40) / 16777216.0 for i in range(n)], np.float32)
        return (u * np.float32(scale) + np.float32(offset)).astype(np.float64)

    def mat(self, name, fmt, rows, cols, sigma=0.02):
        vals = O.synthetic_values(self._seed(name), 0, rows * cols, sigma).reshape(rows, cols)
        if fmt == O.BF16:
            bits = (vals.view(np.uint32) + 0x7FFF + ((vals.view(np.uint32) >> 16) & 1)) >> 16
            return (bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
        return O.Weight.quantized(fmt, vals).dequantize().astype(np.float64)


def _rms(x, w, eps):
    return x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * w


def _silu(x):
    return x / (1 + np.exp(-x))


def _q8(x):
    """The cache's quantizer (gpu/quant.rs:161-180) in float64: per 32, the
    scale amax/127 rounded to f16, each value the nearest multiple."""
    b = x.reshape(-1, 32)
    d = np.array([O.from_f16(O.to_f16(float(v))) for v in np.abs(b).max(1) / 127.0])
    q = np.where(d[:, None] > 0, np.round(b / np.where(d > 0, d, 1)[:, None]), 0)
    return (np.clip(q, -127, 127) * d[:, None]).reshape(x.shape)


class Forward64:
    """qwen35 forward_batch / Pass::layer in float64."""

    def __init__(self, cfg, seed, zero_residual=False):
        self.c, W, H = cfg, Weights(seed), cfg["hidden"]
        hd, kd, vd = cfg["head_dim"], cfg["k_heads"] * cfg["state_dim"], cfg["v_heads"] * cfg["state_dim"]
        qd, kvd = cfg["heads"] * hd, cfg["kv_heads"] * hd
        self.layers = []
        for i in range(cfg["layers"]):
            p = f"blk.{i}."
            L = {"attention": (i + 1) % cfg["full_attention_interval"] == 0,
                 "attn_norm": W.vec(p + "attn_norm", H), "mlp_norm": W.vec(p + "post_attention_norm", H),
                 "gate": W.mat(p + "ffn_gate", O.Q4_K, cfg["intermediate"], H),
                 "up": W.mat(p + "ffn_up", O.Q4_K, cfg["intermediate"], H),
                 "down": W.mat(p + "ffn_down", O.Q4_K, H, cfg["intermediate"])}
            if L["attention"]:
                L.update(q=W.mat(p + "attn_q", O.Q4_K, qd, H), qgate=W.mat(p + "attn_q_gate", O.Q4_K, qd, H),
                         k=W.mat(p + "attn_k", O.Q4_K, kvd, H), v=W.mat(p + "attn_v", O.Q4_K, kvd, H),
                         o=W.mat(p + "attn_output", O.Q4_K, H, qd),
                         q_norm=W.vec(p + "attn_q_norm", hd), k_norm=W.vec(p + "attn_k_norm", hd),
                         kc=np.zeros((0, kvd)), vc=np.zeros((0, kvd)))
            else:
                ch = 2 * kd + vd
                L.update(qkv=W.mat(p + "attn_qkv", O.Q4_K, ch, H), z=W.mat(p + "attn_gate", O.Q4_K, vd, H),
                         ab=W.mat(p + "ssm_ab", O.BF16, 2 * cfg["v_heads"], H),
                         conv=W.vec(p + "ssm_conv1d", ch * 4, 0.3, 0.0).reshape(ch, 4),
                         a=W.uniform(p + "ssm_a", cfg["v_heads"], -0.9, -0.1),
                         dt=W.uniform(p + "ssm_dt.bias", cfg["v_heads"], 8.0, -4.0),
                         norm=W.vec(p + "ssm_norm", cfg["state_dim"]),
                         out=W.mat(p + "ssm_out", O.Q4_K, H, vd),
                         window=np.zeros((3, ch)),
                         S=np.zeros((cfg["v_heads"], cfg["state_dim"], cfg["state_dim"])))
            if zero_residual:
                L["down"] = L["down"] * 0
                L["o" if L["attention"] else "out"] = L["o" if L["attention"] else "out"] * 0
            self.layers.append(L)
        self.norm = W.vec("output_norm", H)
        self.head = W.mat("output", O.Q6_K, cfg["vocab"], H)
        self.embd = W.mat("token_embd", O.Q4_K, cfg["vocab"], H, 1.0)

    def rope(self, x, pos, heads):
        c = self.c
        hd, rot = c["head_dim"], c["rot_dim"]
        x = x.reshape(x.shape[0], heads, hd).copy()
        i = np.arange(rot // 2)
        for t in range(x.shape[0]):
            ang = (pos + t) * float(np.float32(c["rope_theta"])) ** (-(2.0 * i) / rot)
            a, b = x[t, :, i].T.copy(), x[t, :, i + rot // 2].T.copy()
            x[t, :, i] = (a * np.cos(ang) - b * np.sin(ang)).T
            x[t, :, i + rot // 2] = (b * np.cos(ang) + a * np.sin(ang)).T
        return x.reshape(x.shape[0], -1)

    def layer(self, L, x, pos):
        c, eps = self.c, self.c["eps"]
        n = x.shape[0]
        xh = _rms(x, L["attn_norm"], eps)
        if L["attention"]:
            hd, nh, nkv = c["head_dim"], c["heads"], c["kv_heads"]
            q = _rms((xh @ L["q"].T).reshape(n, nh, hd), L["q_norm"], eps).reshape(n, -1)
            k = _rms((xh @ L["k"].T).reshape(n, nkv, hd), L["k_norm"], eps).reshape(n, -1)
            gate, v = xh @ L["qgate"].T, xh @ L["v"].T
            q, k = self.rope(q, pos, nh), self.rope(k, pos, nkv)
            L["kc"] = np.concatenate([L["kc"], _q8(k)])
            L["vc"] = np.concatenate([L["vc"], _q8(v)])
            K, V = L["kc"].reshape(-1, nkv, hd), L["vc"].reshape(-1, nkv, hd)
            att = np.zeros((n, nh, hd))
            for t in range(n):
                for h in range(nh):
                    g = h // (nh // nkv)
                    s = K[:pos + t + 1, g] @ q[t].reshape(nh, hd)[h] / math.sqrt(hd)
                    p = np.exp(s - s.max())
                    att[t, h] = (p / p.sum()) @ V[:pos + t + 1, g]
            x = x + (att.reshape(n, -1) / (1 + np.exp(-gate))) @ L["o"].T
        else:
            d, nk, nv = c["state_dim"], c["k_heads"], c["v_heads"]
            kd = nk * d
            qkv, z, ab = xh @ L["qkv"].T, xh @ L["z"].T, xh @ L["ab"].T
            seq = np.concatenate([L["window"], qkv])
            acc = np.stack([(seq[t:t + 4] * L["conv"].T).sum(0) for t in range(n)])
            L["window"] = seq[-3:]
            y = _silu(acc)
            q = y[:, :kd].reshape(n, nk, d)
            k = y[:, kd:2 * kd].reshape(n, nk, d)
            v = y[:, 2 * kd:].reshape(n, nv, d)
            q = q / np.sqrt((q * q).sum(-1, keepdims=True) + eps)
            k = k / np.sqrt((k * k).sum(-1, keepdims=True) + eps)
            o = np.zeros((n, nv, d))
            for t in range(n):
                for h in range(nv):
                    kh = h // (nv // nk)
                    u = ab[t, h] + L["dt"][h]
                    g = math.exp(L["a"][h] * (u if u > 20 else math.log1p(math.exp(u))))
                    beta = 1 / (1 + math.exp(-ab[t, nv + h]))
                    S = L["S"][h] * g
                    S += np.outer(k[t, kh], (v[t, h] - S.T @ k[t, kh]) * beta)
                    L["S"][h] = S
                    o[t, h] = S.T @ q[t, kh] / math.sqrt(d)
            o = _rms(o, L["norm"], eps).reshape(n, -1)
            x = x + (_silu(z) * o) @ L["out"].T
        xh = _rms(x, L["mlp_norm"], eps)
        return x + (_silu(xh @ L["gate"].T) * (xh @ L["up"].T)) @ L["down"].T

    def forward(self, tokens, pos):
        x = self.embd[np.asarray(tokens)]
        for L in self.layers:
            x = self.layer(L, x, pos)
        return _rms(x[-1], self.norm, self.c["eps"]) @ self.head.T


SEED = 42


def _rel(got, want):
    return np.abs(got - want).max() / np.abs(want).max()


def test_oracle_forward_matches_a_float64_restatement():
    o = O.Model(TINY, SEED)
    f = Forward64(TINY, SEED)
    for tokens, pos in (([3, 17, 42, 7, 9], 0), ([11], 5), ([60, 1, 33], 6), ([2], 9)):
        got, want = o.forward(tokens, pos), f.forward(tokens, pos)
        assert _rel(got, want) < 1e-4, (tokens, pos, _rel(got, want))


def test_restatement_detects_a_swapped_gate_and_up():
    """The check has teeth: the float64 forward with gate and up exchanged in
    one layer differs from the oracle far beyond the tolerance."""
    o = O.Model(TINY, SEED)
    f = Forward64(TINY, SEED)
    L = f.layers[1]
    L["gate"], L["up"] = L["up"], L["gate"]
    assert _rel(o.forward([3, 17, 42, 7, 9], 0), f.forward([3, 17, 42, 7, 9], 0)) > 1e-2


def test_zero_residual_products_leave_head_of_normed_embedding():
    o = O.Model(TINY, SEED)
    o.zero_residual_writes()
    f = Forward64(TINY, SEED)
    for tokens, pos in (([3, 17, 42, 7, 9], 0), ([11], 5)):
        got = o.forward(tokens, pos)
        want = _rms(f.embd[tokens[-1]], f.norm, 1e-6) @ f.head.T
        assert _rel(got, want) < 1e-5
