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
* the state carried across calls (the conv window and the delta-rule state);
* the nextn drafter (Pass::drafter, :663-698): the token's embedding normed by
  enorm and the carried hidden state by hnorm, eh_proj's embedding half and
  hidden half added, one full-attention layer with its own cache, then
  shared_head_norm and the model's head; the draft chain (:1045-1071, each
  later draft fed the drafter's own output), verify (:1073-1091: the linear
  layers' states run apart) and rewind (:1099-1169: the states committed or
  run again over the tokens kept, the drafter catching up from the hidden
  states of the kept tokens).

A slip in the oracle's order (gate and up swapped, the two norms swapped, a
stale conv state; enorm and hnorm exchanged, eh_proj's halves exchanged, the
draft chain fed the carried state) moves the logits far beyond the 1e-4 this
allows: the has-teeth tests make each such slip in the restatement.  A second
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


MAX_DRAFTS = 8  # inference/qwen35/mod.rs:26


class Forward64:
    """qwen35 forward_batch / Pass::layer / Pass::drafter / draft / verify /
    rewind in float64 (inference/qwen35/mod.rs:425-496, 541-698, 1045-1169)."""

    def __init__(self, cfg, seed, zero_residual=False, max_len=64):
        self.c, self.W, self.max_len = cfg, Weights(seed), max_len
        H = cfg["hidden"]
        self.layers = [self._layer(i, (i + 1) % cfg["full_attention_interval"] == 0, zero_residual)
                       for i in range(cfg["layers"])]
        W = self.W
        self.norm = W.vec("output_norm", H)
        self.head = W.mat("output", O.Q6_K, cfg["vocab"], H)
        self.embd = W.mat("token_embd", O.Q4_K, cfg["vocab"], H, 1.0)
        # the nextn drafter (mod.rs:276-288, 379-398): blk.<layers>.*, one full
        # attention layer with a cache of its own; eh_proj's embedding half
        # and hidden half kept apart
        self.drafter = None
        if cfg.get("drafter"):
            p = f"blk.{cfg['layers']}."
            self.drafter = dict(enorm=W.vec(p + "enorm", H), hnorm=W.vec(p + "hnorm", H),
                                eproj=W.mat(p + "eh_proj.embed", O.Q4_K, H, H),
                                hproj=W.mat(p + "eh_proj.hidden", O.Q4_K, H, H),
                                layer=self._layer(cfg["layers"], True, False),
                                dnorm=W.vec(p + "shared_head_norm", H))
        self.carry = None      # the normalized hidden state carried over (State::carry_over)
        self.verified = None   # (tokens, pos, normalized hidden rows) of a batch being verified

    def _layer(self, i, attention, zero_residual):
        cfg, W, H = self.c, self.W, self.c["hidden"]
        hd, kd, vd = cfg["head_dim"], cfg["k_heads"] * cfg["state_dim"], cfg["v_heads"] * cfg["state_dim"]
        qd, kvd = cfg["heads"] * hd, cfg["kv_heads"] * hd
        p = f"blk.{i}."
        L = {"attention": attention,
             "attn_norm": W.vec(p + "attn_norm", H), "mlp_norm": W.vec(p + "post_attention_norm", H),
             "gate": W.mat(p + "ffn_gate", O.Q4_K, cfg["intermediate"], H),
             "up": W.mat(p + "ffn_up", O.Q4_K, cfg["intermediate"], H),
             "down": W.mat(p + "ffn_down", O.Q4_K, H, cfg["intermediate"])}
        if attention:
            L.update(q=W.mat(p + "attn_q", O.Q4_K, qd, H), qgate=W.mat(p + "attn_q_gate", O.Q4_K, qd, H),
                     k=W.mat(p + "attn_k", O.Q4_K, kvd, H), v=W.mat(p + "attn_v", O.Q4_K, kvd, H),
                     o=W.mat(p + "attn_output", O.Q4_K, H, qd),
                     q_norm=W.vec(p + "attn_q_norm", hd), k_norm=W.vec(p + "attn_k_norm", hd),
                     kc=np.zeros((self.max_len, kvd)), vc=np.zeros((self.max_len, kvd)))
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
            L["o" if attention else "out"] = L["o" if attention else "out"] * 0
        return L

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

    def _linear(self, L, qkv, ab, window, S):
        """conv (cpu.rs:250-296), l2 norms, the gated delta rule (cpu.rs:
        298-363) from `window` and `S` (not modified): (o, window, S) after."""
        c, eps = self.c, self.c["eps"]
        n = qkv.shape[0]
        d, nk, nv = c["state_dim"], c["k_heads"], c["v_heads"]
        kd = nk * d
        seq = np.concatenate([window, qkv])
        acc = np.stack([(seq[t:t + 4] * L["conv"].T).sum(0) for t in range(n)])
        y = _silu(acc)
        q = y[:, :kd].reshape(n, nk, d)
        k = y[:, kd:2 * kd].reshape(n, nk, d)
        v = y[:, 2 * kd:].reshape(n, nv, d)
        q = q / np.sqrt((q * q).sum(-1, keepdims=True) + eps)
        k = k / np.sqrt((k * k).sum(-1, keepdims=True) + eps)
        S = S.copy()
        o = np.zeros((n, nv, d))
        for t in range(n):
            for h in range(nv):
                kh = h // (nv // nk)
                u = ab[t, h] + L["dt"][h]
                g = math.exp(L["a"][h] * (u if u > 20 else math.log1p(math.exp(u))))
                beta = 1 / (1 + math.exp(-ab[t, nv + h]))
                Sh = S[h] * g
                Sh += np.outer(k[t, kh], (v[t, h] - Sh.T @ k[t, kh]) * beta)
                S[h] = Sh
                o[t, h] = Sh.T @ q[t, kh] / math.sqrt(d)
        return o, seq[-3:], S

    def layer(self, L, x, pos, verify=False):
        c, eps = self.c, self.c["eps"]
        n = x.shape[0]
        xh = _rms(x, L["attn_norm"], eps)
        if L["attention"]:
            hd, nh, nkv = c["head_dim"], c["heads"], c["kv_heads"]
            q = _rms((xh @ L["q"].T).reshape(n, nh, hd), L["q_norm"], eps).reshape(n, -1)
            k = _rms((xh @ L["k"].T).reshape(n, nkv, hd), L["k_norm"], eps).reshape(n, -1)
            gate, v = xh @ L["qgate"].T, xh @ L["v"].T
            q, k = self.rope(q, pos, nh), self.rope(k, pos, nkv)
            # the cache's positions [pos, pos + n) written over (gpu/mod.rs store)
            L["kc"][pos:pos + n] = _q8(k)
            L["vc"][pos:pos + n] = _q8(v)
            K, V = L["kc"][:pos + n].reshape(-1, nkv, hd), L["vc"][:pos + n].reshape(-1, nkv, hd)
            att = np.zeros((n, nh, hd))
            for t in range(n):
                for h in range(nh):
                    g = h // (nh // nkv)
                    s = K[:pos + t + 1, g] @ q[t].reshape(nh, hd)[h] / math.sqrt(hd)
                    p = np.exp(s - s.max())
                    att[t, h] = (p / p.sum()) @ V[:pos + t + 1, g]
            x = x + (att.reshape(n, -1) / (1 + np.exp(-gate))) @ L["o"].T
        else:
            qkv, z, ab = xh @ L["qkv"].T, xh @ L["z"].T, xh @ L["ab"].T
            o, window, S = self._linear(L, qkv, ab, L["window"], L["S"])
            if verify:
                # mod.rs:606-632: the inputs saved, the states run apart
                L["saved"] = (qkv, ab, L["window"], L["S"])
                L["pending"] = (window, S)
            else:
                L["window"], L["S"] = window, S
            o = _rms(o, L["norm"], eps).reshape(n, -1)
            x = x + (_silu(z) * o) @ L["out"].T
        xh = _rms(x, L["mlp_norm"], eps)
        return x + (_silu(xh @ L["gate"].T) * (xh @ L["up"].T)) @ L["down"].T

    def _body(self, tokens, pos, verify=False):
        x = self.embd[np.asarray(tokens)]
        for L in self.layers:
            x = self.layer(L, x, pos, verify)
        return x

    def run_drafter(self, hidden, tokens, pos):
        """Pass::drafter (mod.rs:663-698): rows of normalized hidden state and
        the tokens that followed them, from position `pos`; returns the
        drafter's output normalized by shared_head_norm."""
        D, eps = self.drafter, self.c["eps"]
        e = _rms(self.embd[np.asarray(tokens)], D["enorm"], eps)
        h = _rms(np.asarray(hidden), D["hnorm"], eps)
        x = e @ D["eproj"].T + h @ D["hproj"].T
        x = self.layer(D["layer"], x, pos)
        return _rms(x, D["dnorm"], eps)

    def forward(self, tokens, pos):
        x = self._body(tokens, pos)
        if self.drafter is None:
            return _rms(x[-1], self.norm, self.c["eps"]) @ self.head.T
        Hn = _rms(x, self.norm, self.c["eps"])
        # the drafter catches up at every position whose next token is known
        # (mod.rs:476-490): from the row carried over, if any
        if self.carry is not None:
            rows, first = np.concatenate([self.carry[None], Hn[:-1]]), 0
        else:
            rows, first = Hn[:-1], 1
        if len(rows):
            self.run_drafter(rows, list(tokens)[first:], pos + first - 1)
        self.carry = Hn[-1]
        return Hn[-1] @ self.head.T

    def draft(self, token, pos, k):
        """LanguageModel::draft (mod.rs:1045-1071): the drafts and the logits
        each was picked from."""
        if self.drafter is None or self.carry is None or self.verified is not None or pos == 0:
            return [], []
        k = min(k, MAX_DRAFTS, max(self.max_len - pos - 1, 0))
        hidden, nxt, drafts, logits = self.carry, token, [], []
        for i in range(k):
            out = self.run_drafter(hidden[None], [nxt], pos - 1 + i)[0]
            lg = out @ self.head.T
            nxt = int(np.argmax(lg))
            drafts.append(nxt)
            logits.append(lg)
            hidden = out
        return drafts, logits

    def verify(self, tokens, pos):
        x = self._body(tokens, pos, verify=True)
        Hn = _rms(x, self.norm, self.c["eps"])
        self.verified = (list(tokens), pos, Hn)
        return Hn @ self.head.T

    def rewind(self, keep):
        """LanguageModel::rewind (mod.rs:1099-1169)."""
        tokens, at, Hn = self.verified
        self.verified = None
        for L in self.layers:
            if L["attention"]:
                continue
            if keep == len(tokens):
                L["window"], L["S"] = L["pending"]
            else:
                qkv, ab, window, S = L["saved"]
                _, L["window"], L["S"] = self._linear(L, qkv[:keep], ab[:keep], window, S)
        if self.drafter is not None:
            rows = np.concatenate([self.carry[None], Hn[:keep - 1]])
            self.run_drafter(rows, tokens[:keep], at - 1)
            self.carry = Hn[keep - 1]


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


DRAFT = dict(TINY, drafter=1)


def _drafts_agree(o, f, token, pos, k, what):
    """The oracle's drafts and the logits of each (drafted again for 1..k,
    since a draft leaves the carried state as it was) against float64's."""
    want, logits = f.draft(token, pos, k)
    got = [int(t) for t in o.draft(token, pos, k)]
    assert got == want, (what, got, want)
    for i in range(len(want)):
        o.draft(token, pos, i + 1)
        assert _rel(o.last_logits(), logits[i]) < 1e-4, (what, i, _rel(o.last_logits(), logits[i]))
    return want


def _speculative_steps(o, f):
    """forward; a draft chain of 3; verify; rewind keeping 2 (the linear
    states run again from the inputs saved, the drafter catching up); a
    draft; verify; rewind keeping all; one more token and a draft."""
    prompt = [3, 17, 42, 7, 9, 30, 2]
    pos = len(prompt)
    assert _rel(o.forward(prompt, 0), f.forward(prompt, 0)) < 1e-4
    d = _drafts_agree(o, f, 11, pos, 3, "first chain")
    batch = [11] + d
    assert _rel(o.verify(batch, pos), f.verify(batch, pos)) < 1e-4
    o.rewind(2)
    f.rewind(2)
    pos += 2
    d = _drafts_agree(o, f, 5, pos, 3, "after a rewind keeping 2")
    batch = [5] + d
    assert _rel(o.verify(batch, pos), f.verify(batch, pos)) < 1e-4
    o.rewind(4)
    f.rewind(4)
    pos += 4
    assert _rel(o.forward([40], pos), f.forward([40], pos)) < 1e-4
    _drafts_agree(o, f, 21, pos + 1, 3, "after a whole batch kept and a token")


def test_oracle_drafter_matches_a_float64_restatement():
    """Pass::drafter, the draft chain (each later draft fed the drafter's own
    output), verify and rewind with the drafter's catch-up, against float64."""
    _speculative_steps(O.Model(DRAFT, SEED), Forward64(DRAFT, SEED))


@pytest.mark.parametrize("swap", ["enorm/hnorm", "eh_proj halves", "hidden fed to chain"])
def test_drafter_restatement_has_teeth(swap):
    """Each slip, made in the float64 restatement, moves the drafts' logits far
    beyond the tolerance: the two input norms exchanged, the two halves of
    eh_proj exchanged, or the chain fed the carried hidden state instead of
    the drafter's own output."""
    o, f = O.Model(DRAFT, SEED), Forward64(DRAFT, SEED)
    D = f.drafter
    if swap == "enorm/hnorm":
        D["enorm"], D["hnorm"] = D["hnorm"], D["enorm"]
    elif swap == "eh_proj halves":
        D["eproj"], D["hproj"] = D["hproj"], D["eproj"]
    prompt = [3, 17, 42, 7, 9, 30, 2]
    o.forward(prompt, 0)
    f.forward(prompt, 0)
    if swap == "hidden fed to chain":
        carried = f.carry
        hidden, nxt = carried, 11
        logits = []
        for i in range(2):
            out = f.run_drafter(hidden[None], [nxt], len(prompt) - 1 + i)[0]
            logits.append(out @ f.head.T)
            nxt = int(np.argmax(logits[-1]))
            hidden = carried
        o.draft(11, len(prompt), 2)
        assert _rel(o.last_logits(), logits[1]) > 1e-2
        return
    _, logits = f.draft(11, len(prompt), 1)
    o.draft(11, len(prompt), 1)
    assert _rel(o.last_logits(), logits[0]) > 1e-2
