"""Writes tests/golden/qwen35_27b_greedy.npz: the oracle's greedy decode of the
random-init 27B-shape model that bench.py runs (64 layers,
hidden 5120, SwiGLU 17408, vocab 248320, Q4_K body, Q6_K head, model seed
1234), after a 4096-token prompt of uniform ids (numpy default_rng(5), as
bench.py draws it).

Per step (the prompt's last position, then each decode token fed back) it
stores the oracle's greedy token, the gap between its two largest logits, the
8 largest logits with their ids, and the logits at 512 fixed vocabulary ids.
The GPU test feeds the oracle's tokens (teacher forcing) and checks its greedy
token wherever the gap exceeds the tolerance, and the logits it stores within
2e-2.

The oracle (oracle/, the C restatement of dwim gpu/cpu.rs and
inference/qwen35/mod.rs) runs on this container's CPUs: about 45 minutes for
the prefill and 3.6 s a decode token on 8 cores.  Usage:
    python tests/golden/make_qwen35_27b_tokens.py [decode_tokens [output.npz]]
"""
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle as O  # noqa: E402

OUT = os.path.join(HERE, "qwen35_27b_greedy.npz")
MODEL_SEED, PROMPT_SEED, PROMPT = 1234, 5, 4096
CFG = dict(hidden=5120, intermediate=17408, layers=64, heads=24, kv_heads=4, head_dim=256, rot_dim=64,
           rope_theta=1e7, full_attention_interval=4, k_heads=16, v_heads=48, state_dim=128, eps=1e-6,
           vocab=248320, drafter=0)


def main():
    steps = int(sys.argv[1]) if len(sys.argv) > 1 else 256
    out = sys.argv[2] if len(sys.argv) > 2 else OUT
    V = CFG["vocab"]
    prompt = np.random.default_rng(PROMPT_SEED).integers(0, V, PROMPT).astype(np.uint32)
    sample = np.sort(np.random.default_rng(77).choice(V, 512, replace=False)).astype(np.uint32)
    t0 = time.time()
    m = O.Model(CFG, MODEL_SEED, O.Q4_K, O.Q6_K, max_len=PROMPT + steps + 8, batch=PROMPT)
    print(f"model built in {time.time() - t0:.0f} s on {O.threads()} threads", flush=True)
    tokens, gaps, top_ids, top_vals, sampled = [], [], [], [], []

    def record(logits):
        order = np.argsort(-logits, kind="stable")[:8]
        tok = int(np.argmax(logits))
        assert tok == int(order[0])
        tokens.append(tok)
        gaps.append(float(logits[order[0]] - logits[order[1]]))
        top_ids.append(order.astype(np.uint32))
        top_vals.append(logits[order].astype(np.float32))
        sampled.append(logits[sample].astype(np.float32))
        np.savez_compressed(out, model_seed=MODEL_SEED, prompt_seed=PROMPT_SEED, prompt=prompt, sample_ids=sample,
                            tokens=np.array(tokens, np.uint32), gaps=np.array(gaps, np.float32),
                            top_ids=np.array(top_ids), top_vals=np.array(top_vals), sampled=np.array(sampled))

    t0 = time.time()
    record(m.forward(prompt, 0))
    print(f"prefill {PROMPT} in {time.time() - t0:.0f} s: token {tokens[-1]} gap {gaps[-1]:.4g}", flush=True)
    for i in range(steps):
        t0 = time.time()
        record(m.forward([tokens[-1]], PROMPT + i))
        print(f"step {i}: token {tokens[-1]} gap {gaps[-1]:.4g} ({time.time() - t0:.1f} s)", flush=True)


if __name__ == "__main__":
    main()
