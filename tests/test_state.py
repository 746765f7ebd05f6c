"""Saving and restoring a sequence's state (LanguageModel::save / restore,
inference/qwen35/mod.rs:905-1017), in the reference's "dwimstat" layout of
version 3, and the carried DeltaNet state of BASELINE config 2 read through
it.

* The oracle and the HIP model follow the reference's test
  `restores_a_saved_state` (:1736-1764): a model restored from the state after
  5 tokens continues exactly as the one that saved it; a state cut short is
  refused.
* The header is spelled out byte by byte from the layout.
* The HIP model's saved bytes round-trip exactly (save, restore, save), and a
  state the oracle saved, restored on the GPU, continues as the oracle does.
* Config 2: one DeltaNet layer at the 27B widths (hidden 5120, 16/48 heads of
  128, Q4_K projections, SwiGLU 17408), its recurrent state seeded N(0, 0.1)
  through restore, runs 1024 single-token steps on the fused decode path; the
  state after steps 1, 16, 256 and 1024 agrees with the oracle's within 1e-3
  of its largest magnitude.
"""
import struct

import numpy as np
import pytest

import oracle as O
from dwim_amd import device as D
from dwim_amd import model as M

SEED = 42


def _header(state):
    magic, version = state[:8], struct.unpack("<I", state[8:12])[0]
    return magic, version, struct.unpack("<7Q", state[12:68])


def _sections(cfg, state):
    """Splits a saved state into (k caches, v caches, conv states, ssm states, hidden)."""
    _, _, (length, caches, slots, kv_dim, conv_w, ssm_w, hidden) = _header(state)
    at, cb = 68, length * kv_dim + length * kv_dim // 32 * 2
    ks = [state[at + i * cb: at + (i + 1) * cb] for i in range(caches)]
    at += caches * cb
    vs = [state[at + i * cb: at + (i + 1) * cb] for i in range(caches)]
    at += caches * cb
    conv, ssm = [], []
    for _ in range(slots):
        conv.append(np.frombuffer(state, np.float32, conv_w, at))
        at += 4 * conv_w
        ssm.append(np.frombuffer(state, np.float32, ssm_w, at))
        at += 4 * ssm_w
    hid = np.frombuffer(state, np.float32, hidden, at) if hidden else None
    assert at + 4 * hidden == len(state)
    return ks, vs, conv, ssm, hid


@pytest.mark.parametrize("drafter", [False, True])
def test_oracle_restores_a_saved_state(drafter):
    cfg = M.config_tiny(drafter).as_dict()
    whole = O.Model(cfg, SEED)
    whole.forward([3, 17, 42, 7, 9], 0)
    state = whole.save(5)
    want = whole.forward([11, 2], 5)
    resumed = O.Model(cfg, SEED)
    assert resumed.restore(state) == 5
    assert np.array_equal(resumed.forward([11, 2], 5), want)
    with pytest.raises(ValueError, match="cut short"):
        resumed.restore(state[:100])
    with pytest.raises(ValueError, match="not a saved state"):
        resumed.restore(b"x" + state[1:])
    with pytest.raises(ValueError, match="another version"):
        resumed.restore(state[:8] + struct.pack("<I", 2) + state[12:])
    other = O.Model(M.config_tiny(not drafter).as_dict(), SEED)
    with pytest.raises(ValueError, match="another model"):
        other.restore(state)


def test_saved_state_header_spelled_out():
    cfg = M.config_tiny(True).as_dict()
    m = O.Model(cfg, SEED, max_len=64)
    m.forward([3, 17, 42, 7, 9], 0)
    state = m.save(5)
    kv_dim, kd, vd = 2 * 256, 2 * 128, 8 * 128
    # magic, version 3, then len, caches (1 attention layer + the drafter's),
    # linear slots (3), kv_dim, conv width 3·(2·k_dim + v_dim), ssm width, hidden
    assert state[:12] == b"dwimstat\x03\x00\x00\x00"
    assert _header(state)[2] == (5, 2, 3, kv_dim, 3 * (2 * kd + vd), 8 * 128 * 128, 1024)
    cb = 5 * kv_dim + 5 * kv_dim // 32 * 2
    assert len(state) == 68 + 2 * 2 * cb + 3 * 4 * (3 * (2 * kd + vd) + 8 * 128 * 128) + 4 * 1024


def test_oracle_has_no_state_to_save_while_verifying_or_before_a_carry():
    cfg = M.config_tiny(True).as_dict()
    m = O.Model(cfg, SEED)
    assert m.save(0) is None  # a drafter, nothing carried over yet
    m.forward([3, 17, 42, 7, 9], 0)
    m.verify([11, 2], 5)
    assert m.save(5) is None
    m.rewind(1)
    assert m.save(6) is not None


@pytest.mark.gpu
@pytest.mark.parametrize("drafter", [False, True])
def test_gpu_restores_a_saved_state(drafter):
    cfg = M.config_tiny(drafter)
    gpu = D.Hip(0)
    whole = M.Model(gpu, cfg, SEED, max_len=64)
    whole.forward([3, 17, 42, 7, 9], 0)
    state = whole.save(5)
    want = whole.forward([11, 2], 5)
    resumed = M.Model(gpu, cfg, SEED, max_len=64)
    assert resumed.restore(state) == 5
    assert resumed.save(5) == state  # byte-exact round trip
    assert np.array_equal(resumed.forward([11, 2], 5), want)
    with pytest.raises(D.DwimError, match="cut short"):
        resumed.restore(state[:100])
    with pytest.raises(D.DwimError, match="another version"):
        resumed.restore(state[:8] + struct.pack("<I", 4) + state[12:])
    # the oracle's state after the same tokens: the same header, caches that
    # agree (Q8 of keys and values within a step), and restored on the GPU it
    # continues as the oracle does
    o = O.Model(cfg.as_dict(), SEED, max_len=64)
    o.forward([3, 17, 42, 7, 9], 0)
    ostate = o.save(5)
    assert _header(ostate) == _header(state)
    g_sec, o_sec = _sections(cfg.as_dict(), state), _sections(cfg.as_dict(), ostate)
    for a, b in zip(g_sec[2] + g_sec[3], o_sec[2] + o_sec[3]):
        assert np.abs(a - b).max() <= 1e-3 * max(1.0, np.abs(b).max())
    for a, b in zip(g_sec[0] + g_sec[1], o_sec[0] + o_sec[1]):
        qa, qb = np.frombuffer(a, np.int8), np.frombuffer(b, np.int8)
        n = len(a) * 32 // 34
        assert np.abs(qa[:n].astype(int) - qb[:n]).max() <= 1
    fresh = M.Model(gpu, cfg, SEED, max_len=64)
    fresh.restore(ostate)
    got, want = fresh.forward([11, 2], 5), o.forward([11, 2], 5)
    assert np.all(np.abs(got - want) <= 2e-3 * (1 + np.abs(want)))
    for m in (whole, resumed, fresh):
        m.close()
    gpu.close()


@pytest.mark.gpu
def test_config2_deltanet_state_over_1024_steps():
    cfg = M.config_27b(False)
    cfg.layers, cfg.vocab = 1, 512
    steps, checks = 1024, (1, 16, 256, 1024)
    gpu = D.Hip(0)
    g = M.Model(gpu, cfg, SEED + 3, max_len=steps + 8)
    o = O.Model(cfg.as_dict(), SEED + 3, max_len=steps + 8, batch=8)
    # a state of no positions: the conv window N(0, 1), the recurrent state N(0, 0.1)
    conv_w, ssm_w = 3 * 10240, 48 * 128 * 128
    header = b"dwimstat" + struct.pack("<I", 3) + struct.pack("<7Q", 0, 0, 1, 1024, conv_w, ssm_w, 0)
    seeded = (header + O.synthetic_values(301, 0, conv_w, 1.0).tobytes() +
              O.synthetic_values(302, 0, ssm_w, 0.1).tobytes())
    assert g.restore(seeded) == 0 and o.restore(seeded) == 0
    tokens = np.random.default_rng(3).integers(0, cfg.vocab, steps)
    for i, t in enumerate(tokens):
        g.forward([int(t)], i, want_logits=False)
        o.forward([int(t)], i)
        if i + 1 in checks:
            gs = _sections(cfg.as_dict(), g.save(i + 1))[3][0]
            os_ = _sections(cfg.as_dict(), o.save(i + 1))[3][0]
            err = np.abs(gs - os_).max() / np.abs(os_).max()
            print(f"step {i + 1}: state max |diff| / max |state| = {err:.2e}", flush=True)
            assert err <= 1e-3, f"step {i + 1}: {err}"
    g.close()
    gpu.close()
