"""BASELINE config 4 at its full size: the random-init 27B-shape model (64
layers, hidden 5120, SwiGLU 17408, vocabulary 248320, Q4_K body, Q6_K head,
model seed 1234) after a 4096-token prompt, then greedy decoding, against the
oracle's run of the same model (tests/golden/qwen35_27b_greedy.npz, written by
tests/golden/make_qwen35_27b_tokens.py from oracle/: the C restatement of
dwim gpu/cpu.rs and inference/qwen35).

As the reference's `gpu_agrees_with_cpu` and its greedy check
(inference/qwen35/mod.rs:1826-1848, :2149), with the north star's bars:
  * teacher-forced (the oracle's token fed back at every step): the logits at
    512 fixed vocabulary ids and the 8 largest within 2e-2 of the oracle's,
    and the greedy token equal to the oracle's wherever the oracle's two
    largest logits are more than 4e-2 apart (twice the logit tolerance, so a
    closer call cannot be decided by it);
  * free-running greedy decoding (dwim_model_forward_greedy, then
    dwim_model_decode_greedy with the device argmax): the same tokens as the
    oracle's, any divergence only at one of its close calls;
  * the prompt fed in pieces of 1 to 65 tokens before the rest: every batch
    class's kernels at the 27B shape, to the same logits after the prompt.
"""
import os

import numpy as np
import pytest

from dwim_amd import device as D
from dwim_amd import model as M

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURE = os.path.join(HERE, "golden", "qwen35_27b_greedy.npz")
LOGIT_TOL, GAP_TOL = 2e-2, 4e-2


@pytest.fixture(scope="module")
def golden():
    if not os.path.exists(FIXTURE):
        pytest.skip("the oracle's fixture has not been generated")
    return np.load(FIXTURE)


@pytest.fixture(scope="module")
def model(golden):
    gpu = D.Hip(0)
    steps = len(golden["tokens"])
    m = M.Model(gpu, M.config_27b(False), int(golden["model_seed"]), D.Q4_K, D.Q6_K,
                max_len=len(golden["prompt"]) + steps + 8)
    yield m
    m.close()
    gpu.close()


def test_teacher_forced_logits_and_tokens_match_the_oracle(golden, model):
    prompt, tokens, gaps = golden["prompt"], golden["tokens"], golden["gaps"]
    ids, top_ids, top_vals, sampled = golden["sample_ids"], golden["top_ids"], golden["top_vals"], golden["sampled"]
    model.reset()
    worst, decided, close = 0.0, 0, 0
    for step in range(len(tokens)):
        if step == 0:
            logits = model.forward(prompt, 0)
        else:
            logits = model.forward([int(tokens[step - 1])], len(prompt) + step - 1)
        err = max(np.abs(logits[ids] - sampled[step]).max(), np.abs(logits[top_ids[step]] - top_vals[step]).max())
        worst = max(worst, float(err))
        assert err <= LOGIT_TOL, f"step {step}: logits differ by {err:.3g}"
        if gaps[step] > GAP_TOL:
            assert int(np.argmax(logits)) == int(tokens[step]), f"step {step}: greedy token"
            decided += 1
        else:
            close += 1
        if step % 16 == 0:
            print(f"step {step}: max |logit diff| {err:.2e} (worst {worst:.2e})", flush=True)
    print(f"{decided} tokens decided and equal, {close} close calls, worst logit diff {worst:.2e}", flush=True)
    assert decided >= 0.8 * len(tokens)


def test_free_running_greedy_tokens_match_the_oracle(golden, model):
    """dwim_model_forward_greedy for the prefill, then dwim_model_decode_greedy
    (each pick handed to the next step on the device) for every step the
    fixture holds: the tokens equal the oracle's until the first step where
    they differ, and that step, if any, is one of the oracle's close calls
    (its two largest logits within 4e-2, which the 2e-2 logit bar leaves
    open); past it the two runs decode different texts."""
    prompt, tokens, gaps = golden["prompt"], golden["tokens"], golden["gaps"]
    model.reset()
    got = [model.forward_greedy(prompt, 0)]
    got += model.decode_greedy(got[0], len(prompt), len(tokens) - 1)
    want = [int(t) for t in tokens]
    diverged = next((i for i in range(len(want)) if got[i] != want[i]), len(want))
    print(f"free-running: {diverged} of {len(want)} tokens equal the oracle's", flush=True)
    if diverged < len(want):
        assert gaps[diverged] <= GAP_TOL, f"step {diverged}: greedy token differs where the oracle decides it"
    first_close = next((i for i, g in enumerate(gaps) if g <= GAP_TOL), len(want))
    assert diverged >= first_close


# The prompt in pieces of the sizes each batch kernel takes (the reference's
# difftest feeds its prompt the same way, testing/difftest/main.rs:96): one
# token (the one-token products and DeltaNet step), 2-4 and 7 (the several-
# token products, runs of up to four), 8-15, 16-17 and 31-33 (the GEMM and the
# token-loop delta rule), 63-65 (the chunked delta rule from 64 on), then the
# rest of the prompt in the model's largest batches.
PIECES = [1, 2, 3, 4, 7, 8, 15, 16, 17, 31, 32, 33, 63, 64, 65]


def test_prompt_fed_in_pieces_reaches_the_oracles_logits(golden, model):
    prompt, ids, top_ids, top_vals, sampled = (golden["prompt"], golden["sample_ids"], golden["top_ids"],
                                               golden["top_vals"], golden["sampled"])
    model.reset()
    pos = 0
    for n in PIECES:
        model.forward(prompt[pos:pos + n], pos, want_logits=False)
        pos += n
    logits = model.forward(prompt[pos:], pos)
    err = max(np.abs(logits[ids] - sampled[0]).max(), np.abs(logits[top_ids[0]] - top_vals[0]).max())
    print(f"pieces {PIECES} + {len(prompt) - pos}: max |logit diff| {err:.2e}", flush=True)
    assert err <= LOGIT_TOL
    if golden["gaps"][0] > GAP_TOL:
        assert int(np.argmax(logits)) == int(golden["tokens"][0])
