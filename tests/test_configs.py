"""Parity at the shapes of the benchmark's configurations:

* config 2, the gated-DeltaNet decode step: hidden 5120, 16 key heads and 48
  value heads of 128, a causal conv of 4 over the q/k/v channels, fp32 state
  48×128×128, Q4_K projections; 1024 consecutive one-token steps through the
  model's fused decode path, the logits after each step against the oracle's
  (the carried state is what they are computed from).  The layer's SwiGLU
  width is cut to 1024, which the configuration does not specify, so that the
  oracle runs the 1024 steps in seconds.
* config 3, GQA attention over the Q8 cache: 24 query heads, 4 key/value
  heads of 256, decode at depths 4096, 32768 and 131072 for two sessions
  (separate caches), and a causal 2048-token prefill at depth 0.

Tolerances as the reference's device checks (gpu/tests.rs:132-140).
"""
import numpy as np
import pytest

import oracle as O
from dwim_amd import device as D
from dwim_amd import model as M

pytestmark = pytest.mark.gpu


def _err(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float((np.abs(got - want) / (1 + np.abs(want))).max())


def test_delta_net_decode_steps_carry_the_state():
    cfg = M.config_27b(False)
    cfg.layers, cfg.vocab, cfg.intermediate = 1, 256, 1024  # layer 0 is a DeltaNet layer
    gpu = D.Hip(0)
    g = M.Model(gpu, cfg, 77, max_len=1100)
    o = O.Model(cfg.as_dict(), 77)
    worst = 0.0
    for step in range(1024):
        token = (step * 37 + 11) % cfg.vocab
        e = _err(g.forward([token], step), o.forward([token], step))
        worst = max(worst, e)
        if step + 1 in (1, 16, 256, 1024):
            print(f"step {step + 1}: max err {e:.2e} (worst so far {worst:.2e})", flush=True)
        assert e <= 2e-3, f"step {step + 1}: {e:.2e}"
    g.close()


@pytest.mark.parametrize("depth", [4096, 32768, 131072])
def test_attention_decode_at_depth_for_two_sessions(depth):
    heads, hd, kvh = 24, 256, 4
    kv_dim = kvh * hd
    gpu = D.Hip(0)
    for session in range(2):
        rng = O.Rng(1000 * session + depth)
        q = rng.floats(heads * hd)
        kd = rng.floats(depth * kv_dim)
        vd = rng.floats(depth * kv_dim)
        want = O.attention(q, O.cache_of(kd, 0), O.cache_of(vd, 0), depth - 1, heads, hd, kvh)
        kc, vc = gpu.alloc_cache(kd.size), gpu.alloc_cache(vd.size)
        gpu.store(kc, 0, gpu.buffer(kd))
        gpu.store(vc, 0, gpu.buffer(vd))
        out = gpu.alloc(heads * hd)
        gpu.attention(out, gpu.buffer(q), kc, vc, depth - 1, heads, hd, kvh)
        e = _err(gpu.read(out), want)
        print(f"depth {depth} session {session}: max err {e:.2e}", flush=True)
        assert e <= 1e-4
    gpu.close()


def test_attention_prefill_of_2048_tokens():
    heads, hd, kvh, n = 24, 256, 4, 2048
    kv_dim = kvh * hd
    rng = O.Rng(2048)
    q = rng.floats(n * heads * hd)
    kd = rng.floats(n * kv_dim)
    vd = rng.floats(n * kv_dim)
    want = O.attention(q, O.cache_of(kd, 0), O.cache_of(vd, 0), 0, heads, hd, kvh)
    gpu = D.Hip(0)
    kc, vc = gpu.alloc_cache(kd.size), gpu.alloc_cache(vd.size)
    gpu.store(kc, 0, gpu.buffer(kd))
    gpu.store(vc, 0, gpu.buffer(vd))
    out = gpu.alloc(q.size)
    gpu.attention(out, gpu.buffer(q), kc, vc, 0, heads, hd, kvh)
    e = _err(gpu.read(out), want)
    print(f"prefill 2048: max err {e:.2e}", flush=True)
    assert e <= 1e-4
    gpu.close()
