"""Workloads for counter runs of single kernels (rocprofv3 --pmc / --kernel-trace).

    python -m dwim_amd.kernel_workloads attention [--reps N]
    python -m dwim_amd.kernel_workloads tokens [--reps N]
    python -m dwim_amd.kernel_workloads stream [--reps N]
    python -m dwim_amd.kernel_workloads verify [--reps N]

`attention`: first a device copy of 256 MiB (four times), the calibration
of the FETCH_SIZE / WRITE_SIZE counters; then one-token GQA decode (24 query heads, 4 key/value heads of 256,
the 27B shape's attention layer) over Q8 caches filled with N(0, 1) keys and
values at context depths 4096, 32768 and 131072, `reps` calls at each depth
(k_attn_partial + k_attn_combine at 4096, k_attn_mfma + k_attn_combine past
6144 positions), and at 32768 `reps` calls of 4 tokens (a verify batch),
each depth's caches distinct; then the same over f16 caches.  Every call goes through the C ABI (dwim_attention).

`tokens`: the 4-token Q4_K product (a speculative-decoding verify batch,
k_planes then k_mv_stream<4>) on the 27B shape's 17408x5120 and 5120x17408
matrices (synthetic weights), `reps` calls each, through dwim_matmul.

`verify`: config 5's verify step.  The 27B-shape model with its MTP drafter
(random-init, Q4_K body, Q6_K head) prefilled with a 32768-token uniform
prompt, then `reps` verify steps of 4 tokens at position 32768, each
rewound to its first token and the model back to its mark (dwim_model_verify,
dwim_model_rewind, dwim_model_rewind_to_mark).

`stream`: the HBM streaming floor the decode products are measured against.
A read and nothing else (dwim_measure_stream, 16 bytes a lane, eight loads
in flight a lane) over 8 distinct buffers of the 17408x5120 product's
50,135,040 weight bytes in turn (400 MB, past the 256 MB Infinity Cache),
launched back to back on the device's stream, `reps` rounds timed with
events, at 256 to 2048 workgroups; prints the read rate.
"""
from __future__ import annotations

import argparse

from . import device as D


def attention(reps: int) -> None:
    dev = D.Hip(0)
    big = 64 << 20  # floats: 256 MiB
    src, dst = dev.alloc(big), dev.alloc(big)
    for _ in range(4):
        dev.copy(dst, 0, src, 0, big)
    dev.sync()
    del src, dst
    heads, hd, kvh = 24, 256, 4
    kv_dim = kvh * hd
    for f16 in (False, True):
        for depth in (4096, 32768, 131072):
            n = depth * kv_dim
            kc = dev.alloc_cache_f16(n) if f16 else dev.alloc_cache(n)
            vc = dev.alloc_cache_f16(n) if f16 else dev.alloc_cache(n)
            dev.store(kc, 0, dev.buffer(D.synthetic_values(depth, 0, n, 1.0)))
            dev.store(vc, 0, dev.buffer(D.synthetic_values(depth + 1, 0, n, 1.0)))
            q = dev.buffer(D.synthetic_values(7, 0, heads * hd, 1.0))
            out = dev.alloc(heads * hd)
            for _ in range(reps):
                dev.attention(out, q, kc, vc, depth - 1, heads, hd, kvh)
            if depth == 32768:
                # a verify batch's 4 tokens at the cache's end
                q4 = dev.buffer(D.synthetic_values(8, 0, 4 * heads * hd, 1.0))
                out4 = dev.alloc(4 * heads * hd)
                for _ in range(reps):
                    dev.attention(out4, q4, kc, vc, depth - 4, heads, hd, kvh)
            dev.sync()
            print(f"attention {'f16' if f16 else 'q8'} depth {depth}: {reps} calls", flush=True)
            del kc, vc
    dev.close()


def tokens(reps: int) -> None:
    dev = D.Hip(0)
    n = 4
    for rows, cols in ((17408, 5120), (5120, 17408)):
        w = dev.upload_synthetic(D.Q4_K, rows, cols, seed=5, sigma=0.02)
        x = dev.buffer(D.synthetic_values(9, 0, n * cols, 1.0))
        out = dev.alloc(n * rows)
        for _ in range(reps):
            dev.matmul(out, w, x)
        dev.sync()
        print(f"tokens {rows}x{cols} n={n}: {reps} calls", flush=True)
        del w, x, out
    dev.close()


def stream(reps: int) -> None:
    import torch

    from . import lib
    from .timing import Event
    nbytes = 17408 * 5120 // 256 * 144
    bufs = [torch.ones(nbytes // 4, device="cuda:0") for _ in range(8)]
    sink = torch.zeros(4, dtype=torch.int32, device="cuda:0")
    torch.cuda.synchronize()
    L = lib()
    dev = D.Hip(0)
    st = dev.stream()
    for blocks in (256, 512, 1024, 2048):
        for i in range(16):
            D._check(L.dwim_measure_stream(dev.h, bufs[i % 8].data_ptr(), nbytes, sink.data_ptr(), blocks))
        dev.sync()
        a, b = Event(), Event()
        a.record(st)
        for i in range(8 * reps):
            D._check(L.dwim_measure_stream(dev.h, bufs[i % 8].data_ptr(), nbytes, sink.data_ptr(), blocks))
        b.record(st)
        us = a.elapsed_ms(b) * 1e3 / (8 * reps)
        print(f"stream: {blocks} blocks, {nbytes} bytes a read in {us:.2f} us = {nbytes / us / 1e6:.2f} TB/s "
              f"({nbytes / us / 1e6 / 8.0:.3f} of 8 TB/s)", flush=True)
    dev.close()


def verify(reps: int) -> None:
    import numpy as np

    from . import model as M
    dev = D.Hip(0)
    prompt_len = 32768
    cfg = M.config_27b(drafter=True)
    model = M.Model(dev, cfg, seed=4321, body_format=D.Q4_K, head_format=D.Q6_K, max_len=prompt_len + 64)
    prompt = np.random.default_rng(55).integers(0, cfg.vocab, prompt_len).astype(np.uint32)
    token = model.forward_greedy(prompt, 0)
    model.mark()
    for _ in range(reps):
        model.verify([token, 1, 2, 3], prompt_len, want_logits=False)
        model.rewind(1)
        model.rewind_to_mark()
    dev.sync()
    print(f"verify: {reps} steps of 4 tokens at {prompt_len}", flush=True)
    model.close()
    dev.close()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("workload", choices=["attention", "tokens", "stream", "verify"])
    ap.add_argument("--reps", type=int, default=20)
    a = ap.parse_args()
    {"attention": attention, "tokens": tokens, "stream": stream, "verify": verify}[a.workload](a.reps)


if __name__ == "__main__":
    main()
