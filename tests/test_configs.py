"""Parity at the shapes of the benchmark's configurations:

* config 2, the gated-DeltaNet decode step, is in test_state.py (its carried
  state, seeded N(0, 0.1), is read back through the saved state);
* config 3, GQA attention: 24 query heads, 4 key/value heads of 256, decode
  at depths 4096, 32768 and 131072 for two sessions (separate caches), and a
  causal 2048-token prefill at depth 0; over the reference's Q8 cache and
  over an f16 cache (the configuration's own wording), each against the
  oracle's attention over the same cache format.

* config 5, the 27B shape with the MTP drafter: two sessions of
  32768-token prompts sharing the weights; speculative decoding (3 drafts,
  verified as a 4-token batch) yields exactly the plain greedy tokens
  (qwen35/mod.rs:2100-2149, inference/local.rs:320-368), and verifying the
  greedy continuation itself as the drafts commits whole batches (rewind with
  keep = 4) and still yields them.

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


def _caches(gpu, kd, vd, f16):
    if f16:
        kc, vc = gpu.alloc_cache_f16(kd.size), gpu.alloc_cache_f16(vd.size)
        want = O.cache_f16_of(kd), O.cache_f16_of(vd)
    else:
        kc, vc = gpu.alloc_cache(kd.size), gpu.alloc_cache(vd.size)
        want = O.cache_of(kd, 0), O.cache_of(vd, 0)
    gpu.store(kc, 0, gpu.buffer(kd))
    gpu.store(vc, 0, gpu.buffer(vd))
    return kc, vc, want


def _oracle_attention(f16, q, kc, vc, pos, heads, hd, kvh):
    return (O.attention_f16 if f16 else O.attention)(q, kc, vc, pos, heads, hd, kvh)


@pytest.mark.parametrize("f16", [False, True], ids=["q8", "f16"])
@pytest.mark.parametrize("depth", [4096, 32768, 131072])
def test_attention_decode_at_depth_for_two_sessions(depth, f16):
    heads, hd, kvh = 24, 256, 4
    kv_dim = kvh * hd
    gpu = D.Hip(0)
    for session in range(2):
        rng = O.Rng(1000 * session + depth)
        q = rng.floats(heads * hd)
        kd = rng.floats(depth * kv_dim)
        vd = rng.floats(depth * kv_dim)
        kc, vc, (ok, ov) = _caches(gpu, kd, vd, f16)
        if f16:
            assert gpu.read_cache(kc, 4096) == ok.read_cache(4096)  # f16 stores are exact
        want = _oracle_attention(f16, q, ok, ov, depth - 1, heads, hd, kvh)
        out = gpu.alloc(heads * hd)
        gpu.attention(out, gpu.buffer(q), kc, vc, depth - 1, heads, hd, kvh)
        e = _err(gpu.read(out), want)
        print(f"depth {depth} session {session} {'f16' if f16 else 'q8'}: max err {e:.2e}", flush=True)
        assert e <= 1e-4
    gpu.close()


@pytest.mark.parametrize("f16", [False, True], ids=["q8", "f16"])
@pytest.mark.parametrize("n", [2, 4, 7, 15])
def test_attention_small_batch_at_depth(n, f16):
    """A verify step's batch (config 5: 4 tokens at 32k): a partial block
    takes up to 4 tokens against the chunk read once; the last chunk holds
    positions of only some of them."""
    heads, hd, kvh = 24, 256, 4
    kv_dim = kvh * hd
    gpu = D.Hip(0)
    for pos in (61, 32766 - n):
        rng = O.Rng(77 * n + pos)
        q = rng.floats(n * heads * hd)
        kd = rng.floats((pos + n) * kv_dim)
        vd = rng.floats((pos + n) * kv_dim)
        kc, vc, (ok, ov) = _caches(gpu, kd, vd, f16)
        want = _oracle_attention(f16, q, ok, ov, pos, heads, hd, kvh)
        out = gpu.alloc(q.size)
        gpu.attention(out, gpu.buffer(q), kc, vc, pos, heads, hd, kvh)
        e = _err(gpu.read(out), want)
        print(f"n {n} pos {pos} {'f16' if f16 else 'q8'}: max err {e:.2e}", flush=True)
        assert e <= 1e-4
    gpu.close()


@pytest.mark.parametrize("f16", [False, True], ids=["q8", "f16"])
def test_attention_prefill_of_2048_tokens(f16):
    heads, hd, kvh, n = 24, 256, 4, 2048
    kv_dim = kvh * hd
    rng = O.Rng(2048)
    q = rng.floats(n * heads * hd)
    kd = rng.floats(n * kv_dim)
    vd = rng.floats(n * kv_dim)
    gpu = D.Hip(0)
    kc, vc, (ok, ov) = _caches(gpu, kd, vd, f16)
    want = _oracle_attention(f16, q, ok, ov, 0, heads, hd, kvh)
    out = gpu.alloc(q.size)
    gpu.attention(out, gpu.buffer(q), kc, vc, 0, heads, hd, kvh)
    e = _err(gpu.read(out), want)
    print(f"prefill 2048 {'f16' if f16 else 'q8'}: max err {e:.2e}", flush=True)
    assert e <= 1e-4
    gpu.close()


def test_f16_cache_round_trips_and_refuses_mixed_formats():
    gpu = D.Hip(0)
    rng = O.Rng(7)
    x = rng.floats(4 * 1024)
    c = gpu.alloc_cache_f16(x.size)
    gpu.store(c, 1024, gpu.buffer(x[1024:]))
    gpu.store(c, 0, gpu.buffer(x[:1024]))
    data = gpu.read_cache(c, x.size)
    assert data == x.astype(np.float16).tobytes()
    c2 = gpu.alloc_cache_f16(x.size)
    gpu.write_cache(c2, data)
    assert gpu.read_cache(c2, x.size) == data
    q8 = gpu.alloc_cache(x.size)
    # a caller sizing its buffer for a Q8 cache (dwim_cache_bytes) is refused
    # for an f16 cache, whose read_cache gives 2 bytes a value
    assert gpu.L.dwim_cache_bytes_of(c.h, x.size) == 2 * x.size
    assert gpu.L.dwim_cache_bytes_of(q8.h, x.size) == gpu.L.dwim_cache_bytes(x.size)
    with pytest.raises(D.DwimError, match="fewer bytes"):
        gpu.read_cache(c, x.size, out_bytes=gpu.L.dwim_cache_bytes(x.size))
    with pytest.raises(D.DwimError, match="different formats"):
        gpu.attention(gpu.alloc(256), gpu.buffer(rng.floats(256)), c, q8, 0, 1, 256, 1)
    gpu.close()


def test_config5_speculative_decoding_equals_greedy_at_size():
    cfg = M.config_27b(drafter=True)
    prompt_len, tokens, k = 32768, 32, 3
    gpu = D.Hip(0)
    model = M.Model(gpu, cfg, seed=4321, max_len=prompt_len + 2 * tokens + 16)
    rng = np.random.default_rng(55)
    seqs = [0, model.add_sequence()]
    firsts = []
    for seq in seqs:  # both sessions prefilled first: their caches coexist
        model.select_sequence(seq)
        firsts.append(model.forward_greedy(rng.integers(0, cfg.vocab, prompt_len).astype(np.uint32), 0))
    for seq, first in zip(seqs, firsts):
        model.select_sequence(seq)
        model.mark()
        plain, token, pos = [], first, prompt_len
        while len(plain) < tokens + k:
            plain.append(token)
            token = model.forward_greedy([token], pos)
            pos += 1
        # speculative, the drafter's own drafts (Local::step with a greedy sampler)
        model.rewind_to_mark()
        spec, token, pos, drafted = [], first, prompt_len, 0
        while len(spec) < tokens:
            spec.append(token)
            drafts = model.draft(token, pos, k)
            drafted += len(drafts)
            _, picks = model.verify([token] + drafts, pos, want_logits=False)
            keep = 1
            for i, d in enumerate(drafts):
                if picks[i] != d:
                    break
                spec.append(d)
                keep += 1
            model.rewind(keep)
            pos += keep
            token = picks[keep - 1]
        print(f"session {seq}: {drafted} drafted, speculative == greedy: {spec[:tokens] == plain[:tokens]}",
              flush=True)
        assert spec[:tokens] == plain[:tokens]
        # the greedy continuation verified as the drafts: every batch kept whole
        model.rewind_to_mark()
        got, token, pos, whole = [], first, prompt_len, 0
        while len(got) < tokens:
            got.append(token)
            drafts = plain[len(got):len(got) + k]
            _, picks = model.verify([token] + drafts, pos, want_logits=False)
            keep = 1
            for i, d in enumerate(drafts):
                if picks[i] != d:
                    break
                got.append(d)
                keep += 1
            whole += keep == len(drafts) + 1
            model.rewind(keep)
            pos += keep
            token = picks[keep - 1]
        print(f"session {seq}: {whole} batches kept whole", flush=True)
        assert got[:tokens] == plain[:tokens]
        assert whole >= 7
    model.close()
    gpu.close()
