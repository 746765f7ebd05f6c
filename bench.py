"""Benchmark: decode and prefill throughput of the 27B-shape Q4_K hybrid qwen35
model on one MI355X, with the roofline of the
dominant decode kernel and the CPU oracle timed on the same host.

A step is one decode token (batch 1) at 4k context: the model is random-init
(synthetic weights of the 27B shape, Q4_K body, Q6_K head, generated on the
device), a 4096-token prompt of uniform random ids is prefilled (timed, as
prefill tok/s), then W untimed and K timed greedy decode steps run.
`value` is decode tokens/s.  The line also carries BASELINE config 5 under
"mtp" (the model with its MTP drafter: two sessions of 32768-token prompts,
greedy speculative decoding against plain greedy decoding from the same
state; --no-mtp skips it).

Prints one JSON line.  --gpus above 1 is refused: this build runs on one GPU.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0


def hip():
    from dwim_amd.timing import hip as h
    L = h()
    vp = ctypes.c_void_p
    L.hipStreamBeginCapture.argtypes = [vp, ctypes.c_int]
    L.hipStreamEndCapture.argtypes = [vp, ctypes.POINTER(vp)]
    L.hipGraphInstantiate.argtypes = [ctypes.POINTER(vp), vp, vp, vp, ctypes.c_size_t]
    L.hipGraphLaunch.argtypes = [vp, vp]
    L.hipGraphExecDestroy.argtypes = [vp]
    L.hipGraphDestroy.argtypes = [vp]
    return L


def graph_us(dev, launch, iters):
    """Average µs of launch(i) for i < iters, captured in a HIP graph so the
    launches follow each other without host gaps, timed with HIP events on
    the device's stream (after two untimed replays)."""
    from dwim_amd.timing import Event
    L = hip()
    st = ctypes.c_void_p(dev.stream())
    graph, execg = ctypes.c_void_p(), ctypes.c_void_p()
    if L.hipStreamBeginCapture(st, 0) != 0:
        raise RuntimeError("hipStreamBeginCapture failed")
    for i in range(iters):
        launch(i)
    if L.hipStreamEndCapture(st, ctypes.byref(graph)) != 0:
        raise RuntimeError("hipStreamEndCapture failed")
    if L.hipGraphInstantiate(ctypes.byref(execg), graph, None, None, 0) != 0:
        raise RuntimeError("hipGraphInstantiate failed")
    L.hipGraphLaunch(execg, st)
    L.hipGraphLaunch(execg, st)
    dev.sync()
    a, b = Event(), Event()
    a.record(st.value)
    L.hipGraphLaunch(execg, st)
    b.record(st.value)
    us = a.elapsed_ms(b) / iters * 1e3
    L.hipGraphExecDestroy(execg)
    L.hipGraphDestroy(graph)
    return us


def kernel_roofline(dev, D, iters=200, copies=8):
    """The decode step's dominant kernel on its own: the feed-forward SwiGLU
    pair (k_mv_q4k_mfma<5>, gate and up 17408x5120 Q4_K in one launch, the
    result's planes handed on), the same launch and grid as in every layer of
    the decode step, which spends about a third of a token in it.  Also the
    single 17408x5120 product.  The token's activations are prepared once
    (int8 planes), then `copies` distinct weights (past the 256 MB Infinity
    Cache) are applied in turn, graph-launched and timed with HIP events.
    Algorithmic bytes per launch: the Q4_K weights (144 B per 256), x and the
    results in f32."""
    rows, cols = 17408, 5120
    x = dev.buffer(D.synthetic_values(9, 0, cols, 1.0))
    out = dev.alloc(rows)
    dev.prepare(x)
    weight_bytes = rows * cols // 256 * 144
    ws = [dev.upload_synthetic(D.Q4_K, rows, cols, seed=100 + i, sigma=0.02) for i in range(2 * copies)]
    pair_us = graph_us(dev, lambda i: dev.swiglu_prepared(out, ws[2 * (i % copies)], ws[2 * (i % copies) + 1]), iters)
    single_us = graph_us(dev, lambda i: dev.matmul_prepared(out, ws[i % copies]), iters)
    del ws
    pair_bytes = 2 * weight_bytes + 4 * cols + 4 * rows
    single_bytes = weight_bytes + 4 * cols + 4 * rows
    return {"kernel": "k_mv_q4k_mfma<5> SwiGLU pair: gate and up 17408x5120 Q4_K, n=1 (int8 MFMA), "
                      "the decode step's feed-forward launch",
            "us": pair_us, "achieved": pair_bytes / (pair_us * 1e-6) / 1e9, "bytes": pair_bytes,
            "single": {"kernel": "k_mv_q4k_mfma<5> Q4_K matvec 17408x5120 n=1 (int8 MFMA)", "us": single_us,
                       "achieved": single_bytes / (single_us * 1e-6) / 1e9, "bytes": single_bytes}}


def stream_floor(dev, reps=50, copies=8, blocks=2048):
    """The box's HBM streaming floor for the roofline kernel's bytes: a read of
    the 17408x5120 product's 50,135,040 weight bytes and nothing else
    (dwim_measure_stream), over `copies` distinct buffers in turn (past the
    Infinity Cache), timed with HIP events on the device's stream; GB/s."""
    import torch
    from dwim_amd import lib
    from dwim_amd.device import _check
    from dwim_amd.timing import Event
    nbytes = 17408 * 5120 // 256 * 144
    bufs = [torch.ones(nbytes // 4, device="cuda:0") for _ in range(copies)]
    sink = torch.zeros(4, dtype=torch.int32, device="cuda:0")
    torch.cuda.synchronize()
    L, st = lib(), dev.stream()
    for i in range(2 * copies):
        _check(L.dwim_measure_stream(dev.h, bufs[i % copies].data_ptr(), nbytes, sink.data_ptr(), blocks))
    dev.sync()
    a, b = Event(), Event()
    a.record(st)
    for i in range(copies * reps):
        _check(L.dwim_measure_stream(dev.h, bufs[i % copies].data_ptr(), nbytes, sink.data_ptr(), blocks))
    b.record(st)
    us = a.elapsed_ms(b) * 1e3 / (copies * reps)
    del bufs
    torch.cuda.empty_cache()
    return nbytes / us / 1e3


def copy_calibration(dev, mib=256, reps=8):
    """A plain device copy of known size (torch's copy kernel, `mib` MiB read
    and written per launch) for scaling the FETCH_SIZE / WRITE_SIZE counters
    of the matvec into bytes."""
    import torch
    n = mib * 1024 * 1024 // 4
    a = torch.ones(n, device="cuda:0")
    b = torch.empty_like(a)
    for _ in range(reps):
        b.copy_(a)
    torch.cuda.synchronize()
    return {"copy_bytes_per_launch": 4 * n}


def measured_traffic(name):
    """HBM bytes per launch of a roofline kernel, from its committed rocprofv3
    PMC passes (FETCH_SIZE, WRITE_SIZE, each scaled by the copy calibration):
    profiles/<name>.json, or None."""
    p = os.path.join(ROOT, "profiles", name + ".json")
    try:
        with open(p) as f:
            return json.load(f)["hbm_bytes_per_launch"]
    except (OSError, KeyError, ValueError):
        return None


def prefill_mfma_counters():
    """MFMA busy of the prefill GEMM from the committed rocprofv3 PMC run
    (profiles/prefill_gemm_mfma.json), or None."""
    p = os.path.join(ROOT, "profiles", "prefill_gemm_mfma.json")
    try:
        with open(p) as f:
            return json.load(f)
    except (OSError, ValueError):
        return None


def prefill_flops(cfg, tokens):
    """Algorithmic flops of a prefill of `tokens` tokens from position 0: 2 per
    weight and token for every body product, the causal attention's
    QK and PV (2·2·heads·head_dim per (query, key) pair with key <= query), and
    the head on the last token."""
    H, F = cfg.hidden, cfg.intermediate
    qd, kvd = cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
    kd, vd = cfg.k_heads * cfg.state_dim, cfg.v_heads * cfg.state_dim
    ffn = 3 * F * H
    lin = (2 * kd + vd) * H + vd * H + 2 * cfg.v_heads * H + H * vd + ffn
    att = (2 * qd + 2 * kvd) * H + H * qd + ffn
    n_att = cfg.layers // cfg.full_attention_interval
    params = (cfg.layers - n_att) * lin + n_att * att
    pairs = tokens * (tokens + 1) // 2
    return 2 * params * tokens + n_att * 4 * cfg.heads * cfg.head_dim * pairs + 2 * cfg.vocab * H


def cpu_prefill_record():
    """The one-time CPU prefill of the same 4096-token prompt on the same
    model, timed when the oracle wrote the config-4 fixture
    (tests/golden/make_qwen35_27b_tokens.py): profiles/cpu_prefill_27b_4096.json,
    or None.  Too long (most of an hour) to rerun in every bench."""
    p = os.path.join(ROOT, "profiles", "cpu_prefill_27b_4096.json")
    try:
        with open(p) as f:
            return json.load(f)
    except (OSError, ValueError):
        return None


def cpu_baseline(cfg, seed, state, tokens, pos0, steps=16):
    """The reference's CPU path on the same workload: the oracle (C
    restatement of dwim gpu/cpu.rs and inference/qwen35, OpenMP over rows and
    heads as rayon does) builds the same random-init model, restores the GPU
    model's saved state after the 4096-token prefill (LanguageModel::restore,
    the dwimstat layout), and decodes `steps` tokens of the same sequence at
    4k context, timed as the reference's token loop would run them.  The
    greedy token after each step is compared with the GPU's."""
    import oracle as O
    t0 = time.time()
    o = O.Model(cfg.as_dict(), seed, O.Q4_K, O.Q6_K, max_len=pos0 + steps + 8, batch=1)
    build_s = time.time() - t0
    assert o.restore(state) == pos0
    agree = 0
    t0 = time.perf_counter()
    for i in range(steps):
        logits = o.forward([int(tokens[i])], pos0 + i)
        agree += int(np.argmax(logits)) == int(tokens[i + 1])
    dt = time.perf_counter() - t0
    del o
    pre = cpu_prefill_record()
    prefill = None
    if pre:
        prefill = {"value": pre["tokens"] / pre["seconds"], "unit": "tok/s", "seconds": pre["seconds"],
                   "cores": pre["threads"], "host": pre["host"], "prompt_sha256": pre["prompt_sha256"],
                   "source": "profiles/cpu_prefill_27b_4096.json: measured once, when the oracle wrote the "
                             "config-4 fixture, not in this run"}
    return {"value": steps / dt, "unit": "tok/s", "cores": O.threads(), "kind": "port", "prefill": prefill,
            "sample": f"C restatement of dwim gpu/cpu.rs + inference/qwen35 (OpenMP), the same 27B-shape model "
                      f"restored from the GPU's state after the 4096-token prefill, {steps} greedy decode tokens "
                      f"at 4k context (model built in {build_s:.0f} s, not timed)",
            "greedy_tokens_equal_to_gpu": f"{agree}/{steps}"}


def mtp_leg(dev, D, M, prompt_len=32768, sessions=2, tokens=64, k=3):
    """the 27B-shape model with a 1-layer MTP drafter,
    `sessions` sessions sharing the weights, each prefilled with a
    `prompt_len`-token uniform-random prompt; then `tokens` tokens of greedy
    speculative decoding (k drafts a step, verified as one (k + 1)-token
    batch: the batch matvecs run on the int8 matrix cores), timed, and from
    the same state (mark / rewind_to_mark) `tokens` tokens of plain greedy
    decoding, timed; the two sequences must be equal (qwen35/mod.rs:2100-2149).
    A step's draft and its verify + rewind are timed apart (the device
    synchronized after the rewind), against a plain token.
    The loop is the reference's Local::step with a greedy sampler
    (inference/local.rs:320-368)."""
    cfg = M.config_27b(drafter=True)
    model = M.Model(dev, cfg, seed=4321, body_format=D.Q4_K, head_format=D.Q6_K, max_len=prompt_len + 2 * tokens + 16)
    rng = np.random.default_rng(55)
    seqs = [0] + [model.add_sequence() for _ in range(sessions - 1)]
    out = {"sessions": sessions, "prompt": prompt_len, "tokens": tokens, "drafts_per_step": k}
    prefill_s = spec_s = plain_s = draft_s = verify_s = 0.0
    accepted = drafted = steps = 0
    match = True
    for seq in seqs:
        model.select_sequence(seq)
        prompt = rng.integers(0, cfg.vocab, prompt_len).astype(np.uint32)
        dev.sync()
        t0 = time.perf_counter()
        first = model.forward_greedy(prompt, 0)
        dev.sync()
        prefill_s += time.perf_counter() - t0
        model.mark()
        # speculative
        t0 = time.perf_counter()
        spec, token, pos = [], first, prompt_len
        while len(spec) < tokens:
            spec.append(token)
            t1 = time.perf_counter()
            drafts = model.draft(token, pos, k)  # (returns the drafts: synchronous)
            t2 = time.perf_counter()
            draft_s += t2 - t1
            steps += 1
            if not drafts:
                token = model.forward_greedy([token], pos)
                pos += 1
                continue
            drafted += len(drafts)
            _, picks = model.verify([token] + drafts, pos, want_logits=False)
            keep = 1
            for i, d in enumerate(drafts):
                if picks[i] != d or len(spec) >= tokens:
                    break
                spec.append(d)
                keep += 1
                accepted += 1
            model.rewind(keep)
            dev.sync()
            verify_s += time.perf_counter() - t2
            pos += keep
            token = picks[keep - 1]
        dev.sync()
        spec_s += time.perf_counter() - t0
        # plain greedy from the same state
        model.rewind_to_mark()
        t0 = time.perf_counter()
        plain, token, pos = [], first, prompt_len
        while len(plain) < tokens:
            plain.append(token)
            token = model.forward_greedy([token], pos)
            pos += 1
        dev.sync()
        plain_s += time.perf_counter() - t0
        match = match and spec[:tokens] == plain
    model.close()
    out.update({"prefill_tok_s": sessions * prompt_len / prefill_s,
                "speculative_tok_s": sessions * tokens / spec_s, "plain_tok_s": sessions * tokens / plain_s,
                "verify_steps": steps, "drafted": drafted, "accepted": accepted,
                "draft_ms": draft_s / steps * 1e3, "verify_rewind_ms": verify_s / steps * 1e3,
                "plain_token_ms": plain_s / (sessions * tokens) * 1e3,
                "verify_over_plain": (verify_s / steps) / (plain_s / (sessions * tokens)),
                "acceptance": accepted / drafted if drafted else 0.0,
                "speculative_equals_greedy": bool(match),
                "note": "random-init drafter: acceptance near zero, so each step yields about one token"})
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=4)
    ap.add_argument("--prompt", type=int, default=4096)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--kernel-only", action="store_true", help="only the decode-matvec roofline leg")
    ap.add_argument("--no-mtp", action="store_true",
                    help="skip the speculative-decoding leg (config 5: MTP drafter, 2 sessions of 32768-token prompts)")
    ap.add_argument("--mtp-prompt", type=int, default=32768)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU; --gpus {args.gpus} is not supported by this build", file=sys.stderr)
        sys.exit(2)

    from dwim_amd import device as D
    from dwim_amd import model as M

    dev = D.Hip(0)
    roof = kernel_roofline(dev, D)
    floor_gbs = stream_floor(dev)
    if args.kernel_only:
        print(json.dumps({"roofline_kernel": roof, "stream_floor_gbs": floor_gbs, "calibration": copy_calibration(dev)}),
              flush=True)
        return

    cfg = M.config_27b(drafter=False)
    max_len = args.prompt + args.warmup + args.steps + 8
    t0 = time.time()
    model = M.Model(dev, cfg, seed=1234, body_format=D.Q4_K, head_format=D.Q6_K, max_len=max_len)
    build_s = time.time() - t0
    rng = np.random.default_rng(5)
    prompt = rng.integers(0, cfg.vocab, args.prompt).astype(np.uint32)

    # prefill: once untimed (first launches load the kernels' code), then
    # from a reset state, timed
    model.forward_greedy(prompt, 0)
    model.reset()
    dev.sync()
    t0 = time.perf_counter()
    tok = model.forward_greedy(prompt, 0)
    dev.sync()
    prefill_s = time.perf_counter() - t0
    pos = args.prompt
    # the state after the prefill, for the CPU baseline (outside any timing)
    state = None if args.no_cpu else model.save(pos)
    decoded = [tok]
    for _ in range(args.warmup):
        tok = model.forward_greedy([tok], pos)
        decoded.append(tok)
        pos += 1
    model.mark()
    start_tok, start_pos = tok, pos
    dev.sync()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        tok = model.forward_greedy([tok], pos)
        decoded.append(tok)
        pos += 1
    dev.sync()
    decode_s = time.perf_counter() - t0
    # the same steps from the same state with the picks fed back on the device
    # (dwim_model_decode_greedy): the host queues every step without waiting
    model.rewind_to_mark()
    dev.sync()
    t0 = time.perf_counter()
    fed = model.decode_greedy(start_tok, start_pos, args.steps)
    dev.sync()
    fed_s = time.perf_counter() - t0
    ms_per_step = decode_s / args.steps * 1e3
    decode_tps = args.steps / decode_s
    # bytes a decode token must read: the Q4_K body, Q6_K head, DeltaNet states
    # (read and written) and the Q8 KV caches at the context depth
    per_layer_ffn = 3 * 17408 * 5120
    lin = 48 * ((10240 + 6144) * 5120 + 5120 * 6144 + per_layer_ffn)
    att = 16 * ((6144 * 2 + 1024 * 2) * 5120 + 5120 * 6144 + per_layer_ffn)
    body = (lin + att) * 144 // 256 + 48 * 96 * 5120 * 2
    head = 248320 * 5120 * 210 // 256
    states = 48 * 2 * (48 * 128 * 128 * 4)
    kv = 16 * 2 * (pos * 1024 * 34 // 32)
    token_bytes = body + head + states + kv
    pf = prefill_flops(cfg, args.prompt)
    counters = prefill_mfma_counters()
    prefill_roofline = {"bound": "mfma", "achieved": pf / prefill_s / 1e12, "peak": 2500.0, "unit": "TFLOP/s",
                        "frac": pf / prefill_s / 1e12 / 2500.0, "algorithmic_flops": pf,
                        "peak_note": "dense f16 MFMA peak of MI355X",
                        # from the committed rocprofv3 PMC run, not measured in this run
                        "gemm_mfma_busy": counters["mfma_busy"] if counters else None,
                        "gemm_mfma_flop_over_algorithmic": counters["mfma_flop_over_algorithmic"] if counters else None,
                        "gemm_mfma_source": "profiles/prefill_gemm_mfma.json (committed rocprofv3 --pmc run of "
                                            "bench.py, not this run)" if counters else None}
    result = {
        "metric": "decode tok/s & prefill tok/s, 27B-shape Q4_K hybrid, 1xMI355X; % HBM peak",
        "value": decode_tps,
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_k weights, f32 activations",
        "data": "synthetic: random-init 27B-shape weights (seeded, generated on the device), uniform random prompt ids",
        "config": {"workload": "27B-shape qwen35 hybrid, prefill 4096 then greedy decode at 4k context",
                   "model": "qwen35-27B-shape", "global_batch": 1, "seq_len": args.prompt,
                   "layers": 64, "hidden": 5120, "ffn": 17408, "vocab": 248320, "weights": "Q4_K body, Q6_K head",
                   "parallelism": "none (1 GPU)"},
        "prefill_tok_s": args.prompt / prefill_s,
        "prefill_s": prefill_s,
        "prefill_roofline": prefill_roofline,
        "decode_device_fed_tok_s": args.steps / fed_s,
        "decode_device_fed_equals_host_loop": fed == decoded[-args.steps:],
        "decode_hbm_frac": token_bytes / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "decode_bytes_per_token": token_bytes,
        "model_build_s": build_s,
        "roofline": {"bound": "hbm", "achieved": roof["achieved"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": roof["achieved"] / HBM_PEAK_GBS,
                     "traffic": measured_traffic("q4k_swiglu_pair_17408x5120_traffic"), "kernel": roof["kernel"],
                     "kernel_us": roof["us"], "algorithmic_bytes": roof["bytes"],
                     # a plain read of one 17408x5120 weight's bytes and nothing else
                     # (dwim_measure_stream), measured in this run
                     "stream_floor_gbs": floor_gbs, "frac_of_stream_floor": roof["achieved"] / floor_gbs,
                     "single_matrix": dict(roof["single"], frac=roof["single"]["achieved"] / HBM_PEAK_GBS,
                                           traffic=measured_traffic("q4k_matvec_17408x5120_traffic"))},
    }
    model.close()
    if not args.no_mtp:
        result["mtp"] = mtp_leg(dev, D, M, prompt_len=args.mtp_prompt)
    if not args.no_cpu and len(decoded) > 16:
        result["cpu_baseline"] = cpu_baseline(cfg, 1234, state, decoded, args.prompt)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
