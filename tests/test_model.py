"""The qwen35 forward pass on the HIP device against the oracle's, on the
reference's tiny synthetic model shape (inference/qwen35/mod.rs:1563-1575) with
the same random weights on both sides (Q4_K body, Q6_K head, bf16 gates).

As the reference's `gpu_agrees_with_cpu` (:1826-1848): logits after a batch of
5 tokens, then 1, then 40, carrying the state, within 2e-3, 2e-3 and 1e-2 of
(1 + |logit|); and, for the greedy decode the benchmark runs, the same tokens
step for step where the oracle's top two logits are apart by more than the
tolerance (a closer call is reported, not failed)."""
import numpy as np
import pytest

import oracle as O
from dwim_amd import device as D
from dwim_amd import model as M

SEED = 42


def _tiny(drafter=True):
    return M.config_tiny(drafter)


def test_oracle_model_is_deterministic_and_sane():
    cfg = _tiny().as_dict()
    a = O.Model(cfg, SEED)
    la = a.forward([3, 17, 42, 7, 9], 0)
    assert np.all(np.isfinite(la)) and np.any(la != 0)
    b = O.Model(cfg, SEED)
    assert np.array_equal(b.forward([3, 17, 42, 7, 9], 0), la)
    assert not np.array_equal(a.forward([11], 5), la)


def test_oracle_model_reset_restores_the_start():
    # qwen35/mod.rs:1736-1764 (the reset half of restores_a_saved_state)
    cfg = _tiny().as_dict()
    m = O.Model(cfg, SEED)
    fresh = m.forward([3, 17, 42, 7, 9], 0)
    m.forward([11, 2], 5)
    assert not np.array_equal(m.forward([3, 17, 42, 7, 9], 7), fresh)
    m.reset()
    assert np.array_equal(m.forward([3, 17, 42, 7, 9], 0), fresh)


def _close(got, want, tol, what):
    bad = np.abs(got - want) > tol * (1 + np.abs(want))
    assert not bad.any(), f"{what}: {got[bad][:4]} vs {want[bad][:4]}"


@pytest.mark.gpu
@pytest.mark.parametrize("drafter", [False, True])
def test_gpu_agrees_with_cpu(drafter):
    cfg = _tiny(drafter)
    gpu = D.Hip(0)
    g = M.Model(gpu, cfg, SEED, max_len=64)
    o = O.Model(cfg.as_dict(), SEED)
    many = [(i * 5 % 43) for i in range(40)]
    for (tokens, pos), tol in zip((([3, 17, 42, 7, 9], 0), ([11], 5), (many, 6)), (2e-3, 2e-3, 1e-2)):
        _close(g.forward(tokens, pos), o.forward(tokens, pos), tol, f"{len(tokens)} tokens at {pos}")
    g.reset()
    o.reset()
    _close(g.forward([3, 17, 42, 7, 9], 0), o.forward([3, 17, 42, 7, 9], 0), 2e-3, "after reset")


@pytest.mark.gpu
def test_greedy_tokens_match_the_oracle():
    cfg = _tiny(False)
    gpu = D.Hip(0)
    g = M.Model(gpu, cfg, SEED + 1, max_len=64)
    o = O.Model(cfg.as_dict(), SEED + 1)
    prompt = [5, 9, 33, 1, 60, 12, 7, 2]
    tok_g = g.forward_greedy(prompt, 0)
    lo = o.forward(prompt, 0)
    tok_o = int(np.argmax(lo))
    close_calls = 0
    for step in range(24):
        top = np.sort(lo)[-2:]
        if top[1] - top[0] > 2e-3 * (1 + abs(top[1])):
            assert tok_g == tok_o, f"step {step}"
        else:
            close_calls += 1
            tok_g = tok_o  # follow the oracle past a near tie
        pos = len(prompt) + step
        tok_g = g.forward_greedy([tok_o], pos)
        lo = o.forward([tok_o], pos)
        tok_o = int(np.argmax(lo))
    assert close_calls <= 2


@pytest.mark.gpu
def test_full_width_layers_agree_with_cpu():
    """The one-token path at the 27B shape's widths (hidden 5120, SwiGLU
    17408, 24/4 attention heads of 256, 16/48 DeltaNet heads of 128): four
    layers (three DeltaNet, one attention) and a 512-token vocabulary, so the
    oracle builds in seconds.  This runs the split products, the planes
    handed between them with their RMS scales, and the fused DeltaNet step
    at their real shapes; the logits after each token agree within 2e-3 of
    (1 + |logit|)."""
    cfg = M.config_27b(False)
    cfg.layers, cfg.vocab = 4, 512
    gpu = D.Hip(0)
    g = M.Model(gpu, cfg, SEED + 2, max_len=32)
    o = O.Model(cfg.as_dict(), SEED + 2)
    _close(g.forward([3, 17, 42, 7, 9], 0), o.forward([3, 17, 42, 7, 9], 0), 2e-3, "5 tokens")
    for i, t in enumerate([11, 400, 2, 77, 301, 5, 64, 128]):
        _close(g.forward([t], 5 + i), o.forward([t], 5 + i), 2e-3, f"token {i}")
    g.close()


@pytest.mark.gpu
def test_one_token_path_with_value_heads_not_a_multiple_of_eight():
    """The fused DeltaNet decode step places a value head's workgroups on one
    XCD when the heads divide by 8, and in order otherwise: 6 value heads over
    2 key heads take the second mapping (the 27B shape's 48 the first)."""
    cfg = _tiny(False)
    cfg.v_heads, cfg.k_heads = 6, 2
    gpu = D.Hip(0)
    g = M.Model(gpu, cfg, SEED + 5, max_len=32)
    o = O.Model(cfg.as_dict(), SEED + 5)
    _close(g.forward([3, 17, 42], 0), o.forward([3, 17, 42], 0), 2e-3, "3 tokens")
    for i, t in enumerate([11, 40, 2, 63, 30]):
        _close(g.forward([t], 3 + i), o.forward([t], 3 + i), 2e-3, f"token {i}")
    g.close()


# ---- drafting, verifying and rewinding (qwen35/mod.rs:1045-1290)

PREFIX, BATCH = [3, 17, 42, 7, 9], [11, 2, 30, 5]
REST = [(i * 5 % 43) for i in range(40)]


def _verify_and_rewind(spec, plain, keep, tol):
    """qwen35/mod.rs:1868-1906: a verified batch's rows are the logits after
    each of its tokens; rewound to `keep` tokens, the model goes on as if it
    had run those alone, and drafts the same."""
    spec.forward(PREFIX, 0)
    plain.forward(PREFIX, 0)
    rows = spec.verify(BATCH, 5)
    if isinstance(rows, tuple):
        rows = rows[0]
    assert rows.shape == (len(BATCH), spec.cfg.vocab if hasattr(spec.cfg, "vocab") else spec.vocab)
    for i, token in enumerate(BATCH[:keep]):
        _close(rows[i], plain.forward([token], 5 + i), tol, f"row {i}")
    spec.rewind(keep)
    at = 5 + keep
    _close(spec.forward([23], at), plain.forward([23], at), tol, "after the rewind")
    assert spec.draft(8, at + 1, 3) == plain.draft(8, at + 1, 3)


@pytest.mark.parametrize("keep", [1, 2, 3, 4])
def test_oracle_verifying_and_rewinding_runs_the_tokens_kept(keep):
    cfg = _tiny().as_dict()
    _verify_and_rewind(O.Model(cfg, SEED), O.Model(cfg, SEED), keep, 1e-4)


def test_oracle_drafts_are_the_drafters_picks():
    # qwen35/mod.rs:1936-1960
    cfg = _tiny().as_dict()
    m = O.Model(cfg, SEED)
    assert m.draft(3, 0, 4) == []
    m.forward(PREFIX, 0)
    drafts = m.draft(11, 5, 4)
    assert len(drafts) == 4 and all(t < cfg["vocab"] for t in drafts)
    assert m.draft(11, 5, 4) == drafts
    assert len(m.draft(11, 5, 100)) == 8
    small = O.Model(cfg, SEED, max_len=8)
    small.forward(PREFIX, 0)
    assert len(small.draft(11, 5, 4)) == 2


def _rewinding(m):
    """qwen35/mod.rs:1772-1791: straight through, with a detour, and with the
    detour taken from a mark rewound to."""
    m.forward(PREFIX, 0)
    straight = (m.forward(REST, 5), m.draft(8, 45, 3))
    m.reset()
    m.forward(PREFIX, 0)
    m.forward([11, 2, 30], 5)
    m.forward([8], 8)
    detoured = (m.forward(REST, 9), m.draft(8, 49, 3))
    m.reset()
    m.forward(PREFIX, 0)
    m.mark()
    m.forward([11, 2, 30], 5)
    m.forward([8], 8)
    m.rewind_to_mark()
    rewound = (m.forward(REST, 5), m.draft(8, 45, 3))
    return straight, detoured, rewound


def test_oracle_rewinds_to_a_mark():
    # qwen35/mod.rs:1793-1824
    cfg = _tiny().as_dict()
    straight, detoured, rewound = _rewinding(O.Model(cfg, SEED))
    assert not np.array_equal(straight[0], detoured[0])
    assert np.array_equal(straight[0], rewound[0])
    assert straight[1] == rewound[1]
    m = O.Model(cfg, SEED)
    with pytest.raises(RuntimeError):
        m.rewind_to_mark()
    m.forward([3, 17], 0)
    m.mark()
    m.reset()
    with pytest.raises(RuntimeError):
        m.rewind_to_mark()


@pytest.mark.gpu
@pytest.mark.parametrize("keep", [1, 3, 4])
def test_verifying_and_rewinding_agrees_with_cpu(keep):
    # qwen35/mod.rs:1919-1934 (2e-2: the batch runs through other kernels
    # than the single tokens it is compared with)
    cfg = _tiny()
    gpu = D.Hip(0)
    _verify_and_rewind(M.Model(gpu, cfg, SEED, max_len=64), M.Model(gpu, cfg, SEED, max_len=64), keep, 2e-2)
    # and against the oracle's own verify
    g = M.Model(gpu, cfg, SEED, max_len=64)
    o = O.Model(cfg.as_dict(), SEED)
    g.forward(PREFIX, 0)
    o.forward(PREFIX, 0)
    rows, greedy = g.verify(BATCH, 5)
    want = o.verify(BATCH, 5)
    for i in range(len(BATCH)):
        _close(rows[i], want[i], 2e-2, f"row {i} against the oracle")
    assert greedy == [int(np.argmax(r)) for r in rows]
    g.rewind(keep)
    o.rewind(keep)
    at = 5 + keep
    _close(g.forward([23], at), o.forward([23], at), 2e-2, "after the rewind, against the oracle")
    assert g.draft(8, at + 1, 3) == o.draft(8, at + 1, 3)


@pytest.mark.gpu
def test_drafts_match_the_oracle():
    cfg = _tiny()
    gpu = D.Hip(0)
    g = M.Model(gpu, cfg, SEED, max_len=64)
    o = O.Model(cfg.as_dict(), SEED)
    assert g.draft(3, 0, 4) == []
    g.forward(PREFIX, 0)
    o.forward(PREFIX, 0)
    drafts = g.draft(11, 5, 4)
    assert drafts == o.draft(11, 5, 4)
    assert g.draft(11, 5, 4) == drafts
    assert len(g.draft(11, 5, 100)) == 8
    small = M.Model(gpu, cfg, SEED, max_len=8)
    small.forward(PREFIX, 0)
    assert len(small.draft(11, 5, 4)) == 2


@pytest.mark.gpu
def test_rewinds_to_a_mark():
    cfg = _tiny()
    gpu = D.Hip(0)
    straight, detoured, rewound = _rewinding(M.Model(gpu, cfg, SEED, max_len=64))
    assert not np.array_equal(straight[0], detoured[0])
    _close(rewound[0], straight[0], 2e-3, "rewound on the GPU")
    assert straight[1] == rewound[1]
    o_straight, _, _ = _rewinding(O.Model(cfg.as_dict(), SEED))
    _close(straight[0], o_straight[0], 1e-2, "against the oracle")
    m = M.Model(gpu, cfg, SEED, max_len=64)
    with pytest.raises(RuntimeError):
        m.rewind_to_mark()
    m.forward([3, 17], 0)
    m.mark()
    m.reset()
    with pytest.raises(RuntimeError):
        m.rewind_to_mark()


@pytest.mark.gpu
def test_sequences_keep_their_own_state():
    # qwen35/mod.rs:1962-2051: two sequences interleaved batch by batch on
    # one model, with a verified draft in one and a mark rewound to in the
    # other, against each run alone on a model of its own (the oracle).
    cfg = _tiny()
    gpu = D.Hip(0)
    o = O.Model(cfg.as_dict(), SEED)
    o.forward(PREFIX, 0)
    first = (o.forward(REST, 5), o.draft(8, 45, 3))
    o.reset()
    o.forward([1, 2, 3, 4], 0)
    second = (o.forward([5, 6], 4), o.draft(7, 6, 3))

    m = M.Model(gpu, cfg, SEED, max_len=64)
    other = m.add_sequence()
    assert other == 1
    m.forward(PREFIX, 0)
    m.select_sequence(other)
    m.forward([1, 2, 3], 0)
    m.select_sequence(0)
    m.mark()
    m.forward([11, 2, 30], 5)
    m.select_sequence(other)
    with pytest.raises(RuntimeError):
        m.rewind_to_mark()  # the mark is the first sequence's
    drafts = m.draft(4, 3, 2)
    assert len(drafts) == 2
    m.verify([4] + drafts, 3)
    with pytest.raises(RuntimeError):
        m.select_sequence(0)  # not while a batch is being verified
    m.rewind(1)
    m.select_sequence(0)
    m.rewind_to_mark()
    got_first = (m.forward(REST, 5), m.draft(8, 45, 3))
    m.select_sequence(other)
    got_second = (m.forward([5, 6], 4), m.draft(7, 6, 3))
    _close(got_first[0], first[0], 1e-2, "the first sequence")
    _close(got_second[0], second[0], 2e-3, "the second sequence")
    assert got_first[1] == first[1]
    assert got_second[1] == second[1]
    with pytest.raises(RuntimeError):
        m.select_sequence(7)


def _greedy(m, prompt, decode):
    out, tok = [], m.forward_greedy(prompt, 0)
    while len(out) < decode:
        out.append(tok)
        tok = m.forward_greedy([tok], len(prompt) + len(out) - 1)
    return out


def _speculative(m, prompt, decode, k=4):
    """The greedy speculative loop of qwen35/mod.rs:2103-2141 (Local::step,
    inference/local.rs:320-368, with a greedy sampler)."""
    toks = list(prompt)
    token = m.forward_greedy(toks, 0)
    out, accepted = [], 0
    while len(out) < decode:
        out.append(token)
        pos = len(toks)
        drafts = m.draft(token, pos, k)
        if not drafts:
            toks.append(token)
            token = m.forward_greedy([token], pos)
            continue
        batch = [token] + drafts
        _, picks = m.verify(batch, pos, want_logits=False)
        keep = 1
        for i, d in enumerate(drafts):
            if picks[i] != d or len(out) >= decode:
                break
            out.append(d)
            keep += 1
            accepted += 1
        m.rewind(keep)
        toks.extend(batch[:keep])
        token = picks[keep - 1]
    return out[:decode], accepted


@pytest.mark.gpu
def test_speculative_decode_is_greedy_decode():
    # qwen35/mod.rs:2100-2149: token for token the same as plain greedy
    cfg = _tiny()
    gpu = D.Hip(0)
    prompt = [5, 9, 33, 1, 60, 12, 7, 2]
    plain = _greedy(M.Model(gpu, cfg, SEED + 2, max_len=64), prompt, 30)
    spec, accepted = _speculative(M.Model(gpu, cfg, SEED + 2, max_len=64), prompt, 30)
    print(f"speculative: {accepted} drafts accepted")
    assert spec == plain


@pytest.mark.gpu
@pytest.mark.parametrize("shape", ["tiny", "tiny+drafter", "27b-widths"])
def test_device_fed_decode_is_greedy_decode(shape):
    """dwim_model_decode_greedy (each step's pick handed to the next step's
    embedding on the device) gives the tokens of the host loop of
    forward_greedy calls, leaves the same state behind (the step after it
    agrees), and on the 27B widths runs the fused one-token path with the
    Q6_K head's planes."""
    if shape == "27b-widths":
        cfg = M.config_27b(False)
        cfg.layers, cfg.vocab = 4, 512
    else:
        cfg = _tiny(shape == "tiny+drafter")
    gpu = D.Hip(0)
    prompt = [5, 9, 33, 1, 60, 12, 7, 2]
    host, dev = M.Model(gpu, cfg, SEED + 3, max_len=64), M.Model(gpu, cfg, SEED + 3, max_len=64)
    want = _greedy(host, prompt, 21)
    first = dev.forward_greedy(prompt, 0)
    assert first == want[0]
    got = [first] + dev.decode_greedy(first, len(prompt), 13)
    got += dev.decode_greedy(got[-1], len(prompt) + 13, 7)
    assert got[:21] == want
    assert dev.decode_greedy(got[-1], len(prompt) + 20, 0) == []
    with pytest.raises(RuntimeError):
        dev.decode_greedy(got[-1], 60, 5)  # past the cache
    with pytest.raises(RuntimeError):
        dev.decode_greedy(cfg.vocab + 10**6, 30, 1)  # past the table
    host.close()
    dev.close()


def _sampled(m, prompt, decode, k, ref_settings, gpu):
    """Local::step / Local::pick (inference/local.rs:299-368) with the
    device sampler picking from the model's device logits: after the prompt
    a pick from the last row; then, token by token, drafts verified as one
    batch, each row's draft checked (Sampler::verify) until one is replaced,
    the batch rewound to the tokens kept.  Every pick and acceptance is also
    made by the oracle's sampler on the same logits read back, and must agree."""
    dev_s = gpu.sampler(*ref_settings)
    ref_s = O.Sampler(*ref_settings)
    vocab = m.cfg.vocab
    m.forward(prompt, 0, want_logits=False)
    buf = m.logits_buffer()
    row = gpu.read(buf)[:vocab]
    token = dev_s.sample(buf, 0, vocab)
    assert token == ref_s.sample(row)
    out, pos, accepted = [], len(prompt), 0
    while len(out) < decode:
        out.append(token)
        drafts = m.draft(token, pos, k)
        if not drafts:
            m.forward([token], pos, want_logits=False)
            buf = m.logits_buffer()
            token, want = dev_s.sample(buf, 0, vocab), ref_s.sample(gpu.read(buf)[:vocab])
            assert token == want
            pos += 1
            continue
        batch = [token] + drafts
        m.verify(batch, pos, want_logits=False)
        buf = m.logits_buffer()
        rows = gpu.read(buf)[:len(batch) * vocab].reshape(len(batch), vocab)
        keep = 1
        for i in range(len(batch)):
            if i < len(drafts):
                got = dev_s.verify(buf, drafts[i], i, vocab)
                assert got == ref_s.verify(rows[i], drafts[i])
                token, ok = got
                if not ok:
                    break
                out.append(token)
                accepted += 1
                keep += 1
            else:
                token = dev_s.sample(buf, i, vocab)
                assert token == ref_s.sample(rows[i])
        m.rewind(keep)
        pos += keep
    assert dev_s.rng == ref_s.rng
    return out[:decode], accepted


@pytest.mark.gpu
@pytest.mark.parametrize("settings", [(1.0, 20, 0.95, 0.05, 17), (0.3, 5, 1.0, 0.0, 3), (0.0, 20, 0.95, 0.05, 1)])
def test_speculative_sampling_with_the_device_sampler(settings):
    cfg = _tiny()
    gpu = D.Hip(0)
    prompt = [5, 9, 33, 1, 60, 12, 7, 2]
    out, accepted = _sampled(M.Model(gpu, cfg, SEED + 2, max_len=96), prompt, 30, 3, settings, gpu)
    print(f"sampled: {accepted} drafts accepted")
    assert len(out) == 30
    if settings[0] == 0.0:
        # at temperature zero sampling is greedy decoding
        assert out == _greedy(M.Model(gpu, cfg, SEED + 2, max_len=96), prompt, 30)
