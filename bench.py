#!/usr/bin/env python3
"""Benchmark of the MI355X speculative verify path (headline metric).

Workload (benchmark config 4): random-init decoder, 32 layers, d_model 4096,
32 query / 8 KV heads (head_dim 128), SwiGLU ffn 11008, vocab 32000; INT4 g128
weights (fp16 scale/zero) drawn N(0, 0.02^2) before quantisation, bf16 tied LM
head, 3 MTP heads (num_future_tokens 4, k = 3 drafts + 1 -> K = 4 verify rows),
INT8 KV cache holding a 4096-token synthetic context per sequence.

A "step" is one speculative round of the MTP engine (mtp_speculative.rs:161-322)
for every sequence of the batch: 3 MTP-head forwards, one K=4-row verify
forward over the 4096-token cache, fused acceptance, replay on rejection.
`value` = committed tokens / wall time of the timed greedy rounds at batch 32
(inputs and KV resident in HBM); batches 1 and 8 are reported beside it, and the
same rounds with the reference CLI's sampler (T 0.7, top-k 50, top-p 0.9) in
`per_batch_sampled_cli`.  The verify
step (K = 4 rows at offset 4096, repeated) is timed separately with per-kernel
HIP events at dispatch level: the INT4 GEMV gives `roofline` (batch 1, HBM), the
decode attention `roofline_attention` (batch 1, HBM) and `roofline_attention_b32`
(batch 32, HBM), and the many-row GEMM `roofline_gemm` (batch 32, MFMA).  Also measured: the standalone sampled
acceptance kernel of config 2 (32 x 4 x 32000, T = 0.8, HBM) and the config-3
INT8 verify step at batch 1 and 16 (HBM).  `cpu_baseline` times the CPU oracle
(restated reference CPU path, f32) on all host cores on a 2-layer slice of the
same model and extrapolates to a full round.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "aarambh-ai_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

import numpy as np  # noqa: E402

METRIC = "accepted tokens/s at batch 1 & 32 (INT4, k=3); verify-step HBM GB/s % of peak"
HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0

C4 = dict(vocab_size=32000, hidden_dim=4096, ffn_dim=11008, n_layers=32, n_heads=32, n_kv_heads=8,
          max_seq_len=4096 + 512, num_future_tokens=4)
CTX = 4096
K_ROWS = 4  # k = 3 MTP drafts + the target-sampled proposal

C3 = dict(vocab_size=32000, hidden_dim=2048, ffn_dim=5632, n_layers=16, n_heads=16, n_kv_heads=4,
          max_seq_len=2048 + 64)
C3_CTX = 2048


def int4_matrix_bytes(n, k):
    return n * k // 2 + n * (k // 128) * 4  # codes + fp16 scale + fp16 zero per 128-group


def int8_matrix_bytes(n, k):
    return n * k + n * 4  # codes + f32 row scale


def layer_shapes(cfg):
    H, F = cfg["hidden_dim"], cfg["ffn_dim"]
    hd = H // cfg["n_heads"]
    QD, KD = cfg["n_heads"] * hd, cfg["n_kv_heads"] * hd
    return [(QD + 2 * KD, H), (H, QD), (2 * F, H), (H, F)], hd


def verify_alg_bytes(B, ctx=CTX):
    """Algorithmic HBM bytes of one K-row verify step at batch B (config 4): every weight
    byte once (quantised, with scales), the LM head once, and per sequence the K / V
    cache bytes of the context at every layer."""
    shapes, hd = layer_shapes(C4)
    per_layer = sum(int4_matrix_bytes(n, k) for n, k in shapes)
    weights = C4["n_layers"] * per_layer + C4["vocab_size"] * C4["hidden_dim"] * 2
    kv = B * C4["n_layers"] * 2 * C4["n_kv_heads"] * ctx * (hd + 2)  # INT8 codes + fp16 per-token scale
    return weights, kv


def c3_alg_bytes(B):
    shapes, hd = layer_shapes(C3)
    weights = C3["n_layers"] * sum(int8_matrix_bytes(n, k) for n, k in shapes) + C3["vocab_size"] * C3["hidden_dim"] * 2
    kv = B * C3["n_layers"] * 2 * C3["n_kv_heads"] * C3_CTX * hd * 2  # fp16 K and V
    return weights, kv


def gemm_flops(M, cfg=C4):
    shapes, _ = layer_shapes(cfg)
    return 2.0 * M * cfg["n_layers"] * sum(n * k for n, k in shapes)


def verify_timing(m, ids, offs, n_iter):
    """Wall time of the verify step as served (captured-graph replay), then per-kernel
    classes from HIP events at each dispatch's start / end (direct launches)."""
    for _ in range(3):
        m.forward_with_cache_output(ids, offs, want_logits=False, want_hidden=False)
    m.sync()
    t = time.perf_counter()
    for _ in range(n_iter):
        m.forward_with_cache_output(ids, offs, want_logits=False, want_hidden=False)
    m.sync()
    wall = (time.perf_counter() - t) / n_iter
    m.prof_enable(True)
    for _ in range(n_iter):
        m.forward_with_cache_output(ids, offs, want_logits=False, want_hidden=False)
    m.sync()
    prof = m.prof_get()
    m.prof_enable(False)
    return wall, prof


def kernels_summary(prof, n):
    return {k: {"ms_per_step": v["ms"] / n, "launches_per_step": v["launches"] / n,
                "gbs": (v["bytes"] / (v["ms"] * 1e-3) / 1e9) if v["ms"] > 0 else 0.0}
            for k, v in prof.items() if v["launches"]}


INT4_CLASSES = ("gemv_qkv", "gemv_wo", "gemv_gateup", "gemv_down")


def run_c4(args):
    import aarambh_hip as A

    cfg = A.ModelConfig(**C4, weight_format=A.W_INT4_G128, lm_head_format=1, kv_format=A.KV_INT8)
    bmax = max(args.batches)
    t0 = time.time()
    m = A.HipModel(cfg, max_batch=bmax, max_rows=128)
    m.init_synthetic(seed=0, std=0.02)
    print(f"# model ready in {time.time() - t0:.1f}s", file=sys.stderr, flush=True)
    eng = A.MtpSpeculativeEngine(m, A.SpeculativeConfig(K_ROWS))
    rng = np.random.default_rng(0)
    res = {}
    _, hd = layer_shapes(C4)
    for B in args.batches:
        for b in range(B):
            m.kv_fill_synthetic(b, CTX, seed=1 + b)
        # ---- verify step: K rows at offset CTX (rewinds each time) ----
        ids = rng.integers(1, C4["vocab_size"], (B, K_ROWS)).astype(np.uint32)
        n_verify = args.verify_iters
        tv, prof = verify_timing(m, ids, [CTX] * B, n_verify)
        wbytes, kvbytes = verify_alg_bytes(B)
        gpu_ms = sum(v["ms"] for v in prof.values()) / n_verify
        # ---- engine rounds ----
        prompts = rng.integers(1, C4["vocab_size"], (B, 1)).astype(np.uint32)
        max_new = K_ROWS * (args.warmup + args.steps + 2) + 8
        sess = eng.session(prompts, max_new, A.Sampler.greedy_sampler(), cached_len=CTX)
        sess.step(args.warmup)
        tok0 = sum(len(r.token_ids) for r in sess.result())
        m.sync()
        ts = time.perf_counter()
        sess.step(args.steps)
        m.sync()
        ts = time.perf_counter() - ts
        after = sess.result()
        tok1 = sum(len(r.token_ids) for r in after)
        stats_all = [r.speculative_stats for r in after]
        sess.close()
        rounds = sum(s.rounds for s in stats_all)
        # the same rounds with the reference CLI's sampler (T 0.7, top-k 50, top-p 0.9,
        # infer.rs:72-77), one seed per sequence
        for b in range(B):
            m.kv_fill_synthetic(b, CTX, seed=1 + b)
        ssess = eng.session(prompts, max_new, A.Sampler.top_k_top_p(0.7, top_k=50, top_p=0.9), cached_len=CTX,
                            seeds=np.arange(B, dtype=np.uint64))
        ssess.step(args.warmup)
        st0 = sum(len(r.token_ids) for r in ssess.result())
        m.sync()
        tss = time.perf_counter()
        ssess.step(args.steps)
        m.sync()
        tss = time.perf_counter() - tss
        sres = ssess.result()
        ssess.close()
        sampled = {"tokens_per_s": (sum(len(r.token_ids) for r in sres) - st0) / tss,
                   "ms_per_step": tss * 1000.0 / args.steps,
                   "acceptance_rate": float(np.mean([r.speculative_stats.acceptance_rate() for r in sres]))}
        int4 = [prof[k] for k in INT4_CLASSES]
        ms4 = sum(v["ms"] for v in int4)
        by4 = sum(v["bytes"] for v in int4)
        n4 = sum(v["launches"] for v in int4)
        att = prof["attention"]
        res[B] = {
            "tokens_per_s": (tok1 - tok0) / ts,
            "ms_per_step": ts * 1000.0 / args.steps,
            "tokens_timed": tok1 - tok0,
            "acceptance_rate": float(np.mean([s.acceptance_rate() for s in stats_all])),
            "tokens_per_round": tok1 / max(1, rounds / B),
            "target_forwards_per_round": sum(s.target_decode_forwards for s in stats_all) / max(1, rounds),
            "mtp_forwards_per_round": sum(s.mtp_head_forwards for s in stats_all) / max(1, rounds),
            "verify": {
                "ms_wall": tv * 1000.0,
                "ms_kernels": gpu_ms,
                "alg_bytes": wbytes + kvbytes,
                "hbm_gbs": (wbytes + kvbytes) / tv / 1e9,
                "hbm_frac": (wbytes + kvbytes) / tv / 1e9 / HBM_PEAK_GBS,
                "kernels": kernels_summary(prof, n_verify),
            },
            "stats_seq0": stats_all[0].__dict__,
            "sampled_cli": sampled,
            "int4_proj": {"ms_per_step": ms4 / n_verify, "alg_bytes": by4, "launches": n4,
                          "avg_us": ms4 * 1000.0 / max(n4, 1), "avg_bytes": by4 / max(n4, 1),
                          "gbs": by4 / (ms4 * 1e-3) / 1e9 if ms4 else 0.0,
                          "useful_tflops": gemm_flops(B * K_ROWS) / (ms4 * 1e-3 / n_verify) / 1e12 if ms4 else 0.0},
            "attention": {"ms_per_step": att["ms"] / n_verify, "launches": att["launches"],
                          "avg_us": att["ms"] * 1000.0 / max(att["launches"], 1),
                          "alg_bytes_per_step": kvbytes,
                          "gbs": kvbytes / (att["ms"] * 1e-3 / n_verify) / 1e9 if att["ms"] else 0.0},
        }
        print(f"# B={B}: {res[B]['tokens_per_s']:.1f} tok/s, round {res[B]['ms_per_step']:.3f} ms, verify "
              f"{tv * 1000:.3f} ms ({res[B]['verify']['hbm_gbs']:.0f} GB/s), int4 proj "
              f"{res[B]['int4_proj']['gbs']:.0f} GB/s / {res[B]['int4_proj']['useful_tflops']:.0f} TF, attention "
              f"{res[B]['attention']['gbs']:.0f} GB/s; sampled (T 0.7, top-k 50, top-p 0.9) "
              f"{sampled['tokens_per_s']:.1f} tok/s, round {sampled['ms_per_step']:.3f} ms", file=sys.stderr, flush=True)
    m.close()
    return res


def run_serve(args):
    """Continuous batching with speculative rounds (the serving worker's loop,
    serve/src/batching.rs:324-445, with decode_sessions replaced by MTP rounds) on the C4
    model: 8 rows, a stream of 24 greedy requests with ragged prompts (64-512 tokens) and
    token budgets (64-192), all queued at the start (a loaded server).  Requests join
    free rows between rounds (prefill in 128-token chunks, the reference's
    prefill_chunk_size) and leave when done.  Committed tokens / wall time of the whole
    stream, admission prefills included; the stream runs once untimed first so that the
    forward graphs of its shapes are captured (a warm server)."""
    import aarambh_hip as A

    cfg = A.ModelConfig(**C4, weight_format=A.W_INT4_G128, lm_head_format=1, kv_format=A.KV_INT8)
    cap, nreq = 8, 24
    m = A.HipModel(cfg, max_batch=cap, max_rows=128)
    m.init_synthetic(seed=0, std=0.02)
    if args.no_graphs:
        m.set_graphs(False)
    eng = A.MtpSpeculativeEngine(m, A.SpeculativeConfig(K_ROWS))
    rng = np.random.default_rng(5)
    reqs = [A.GenerationRequest(rng.integers(1, C4["vocab_size"], int(rng.integers(64, 513))).astype(np.uint32),
                                int(rng.integers(64, 193)), seed=i) for i in range(nreq)]

    def stream():
        bat = A.SpeculativeBatcher(eng, A.BatcherConfig(max_batch_size=cap, queue_capacity=nreq),
                                   A.Sampler.greedy_sampler())
        for r in reqs:
            bat.submit(r)
        steps = 0
        events = []
        m.sync()
        t = time.perf_counter()
        while bat.pending():
            events += bat.step()
            steps += 1
        m.sync()
        t = time.perf_counter() - t
        bat.close()
        done = [e[2] for e in events if e[0] == "completed"]
        assert len(done) == nreq, [e for e in events if e[0] == "failed"]
        return t, steps, done

    stream()
    t, steps, done = stream()
    toks = sum(len(o.token_ids) for o in done)
    st = [o.speculative_stats for o in done]
    rounds = sum(s.rounds for s in st)
    m.close()
    res = {
        "tokens_per_s": toks / t,
        "requests_per_s": nreq / t,
        "wall_s": t,
        "tokens": toks,
        "prompt_tokens": int(sum(len(r.prompt_ids) for r in reqs)),
        "batcher_steps": steps,
        "mean_rows_per_round": rounds / max(steps, 1),
        "acceptance_rate": float(np.mean([s.acceptance_rate() for s in st])),
        "tokens_per_request_round": toks / max(rounds, 1),
    }
    print(f"# serve: {res['tokens_per_s']:.1f} tok/s over {nreq} requests in {t:.2f}s, "
          f"{res['mean_rows_per_round']:.2f} rows per round", file=sys.stderr, flush=True)
    return res


def run_c2(args):
    """benchmark config 2: the standalone fused acceptance kernel, 32 sequences x k = 4
    draft positions x vocab 32000, target logits N(0, 3^2), draft = target + N(0, 1),
    T = 0.8, draft tokens drawn from the draft distribution, seeded uniforms (external-
    draft round with bonus row).  One call reads 36 864 000 bytes of logits."""
    import torch
    import aarambh_hip as A

    B, K, V = 32, 4, 32000
    m = A.HipModel(A.ModelConfig(vocab_size=128, hidden_dim=128, ffn_dim=128, n_layers=1, n_heads=1,
                                 n_kv_heads=1, max_seq_len=16), max_batch=1, max_rows=16)
    g = torch.Generator(device="cuda").manual_seed(0)
    tgt = torch.randn((B, K + 1, V), device="cuda", generator=g) * 3.0
    drf = tgt[:, :K] + torch.randn((B, K, V), device="cuda", generator=g)
    toks = torch.multinomial(torch.softmax(drf.reshape(-1, V) / 0.8, -1), 1, generator=g).reshape(B, K).int()
    seeds = torch.arange(B, device="cuda", dtype=torch.int64)
    s = A.Sampler.top_k_top_p(0.8, seed=0)
    which = getattr(args, "c2_sampler", "both")
    n = args.verify_iters * 5
    alg = B * (2 * K + 1) * V * 4
    us, acc, prof = float("nan"), np.zeros(1), {"launches": 0}
    if which in ("both", "plain"):
        out = None
        for _ in range(3):
            out = m.accept_sample(tgt, drf, toks, s, True, seeds=seeds)
        m.prof_enable(True)
        for _ in range(n):
            m.accept_sample(tgt, drf, toks, s, True, seeds=seeds)
        prof = m.prof_get()["accept"]
        m.prof_enable(False)
        us = prof["ms"] * 1000.0 / max(prof["launches"], 1)
        acc = out["accept_len"].cpu().numpy()
    # the same shape with the reference CLI's sampler (infer.rs:72-77: T 0.7, top-k 50, top-p 0.9);
    # draft tokens from the draft's top-k / top-p set, as the engines propose them
    s_cli = A.Sampler.top_k_top_p(0.7, top_k=50, top_p=0.9, seed=0)
    pv, pi = torch.topk(torch.softmax(drf.reshape(-1, V) / 0.7, -1), 50, dim=-1)
    keep = (torch.cumsum(pv, -1) - pv) < 0.9
    pick = torch.multinomial(pv * keep, 1, generator=g)
    toks_cli = torch.gather(pi, 1, pick).reshape(B, K).int()
    us_cli = float("nan")
    if which in ("both", "cli"):
        for _ in range(3):
            m.accept_sample(tgt, drf, toks_cli, s_cli, True, seeds=seeds)
        m.prof_enable(True)
        for _ in range(n):
            m.accept_sample(tgt, drf, toks_cli, s_cli, True, seeds=seeds)
        prof_cli = m.prof_get()["accept"]
        m.prof_enable(False)
        us_cli = prof_cli["ms"] * 1000.0 / max(prof_cli["launches"], 1)
    m.close()
    r = {"us_per_call": us, "alg_bytes": alg, "gbs": alg / (us * 1e-6) / 1e9, "hbm_frac": alg / (us * 1e-6) / 1e9 /
         HBM_PEAK_GBS, "launches": prof["launches"], "mean_accept_len": float(acc.mean()),
         "cli_sampler_us_per_call": us_cli}
    print(f"# C2 sampled acceptance: {us:.2f} us per call, {r['gbs']:.0f} GB/s; with the CLI sampler "
          f"(T 0.7, top-k 50, top-p 0.9) {us_cli:.2f} us", file=sys.stderr, flush=True)
    return r


def run_c3(args):
    """benchmark config 3: INT8 per-row verify, 16 layers, d 2048, 16 / 4 heads, ffn 5632,
    fp16 KV cache of 2048 tokens, K = 4 rows at batch 1 and 16."""
    import aarambh_hip as A

    cfg = A.ModelConfig(**C3, weight_format=A.W_INT8_ROW, lm_head_format=1, kv_format=A.KV_F16)
    m = A.HipModel(cfg, max_batch=16, max_rows=128)
    m.init_synthetic(seed=0, std=0.02)
    rng = np.random.default_rng(3)
    res = {}
    for B in (1, 16):
        for b in range(B):
            m.kv_fill_synthetic(b, C3_CTX, seed=1 + b)
        ids = rng.integers(1, C3["vocab_size"], (B, K_ROWS)).astype(np.uint32)
        tv, prof = verify_timing(m, ids, [C3_CTX] * B, args.verify_iters)
        w, kv = c3_alg_bytes(B)
        res[B] = {"ms_wall": tv * 1e3, "alg_bytes": w + kv, "hbm_gbs": (w + kv) / tv / 1e9,
                  "hbm_frac": (w + kv) / tv / 1e9 / HBM_PEAK_GBS, "kernels": kernels_summary(prof, args.verify_iters)}
        print(f"# C3 B={B}: verify {tv * 1e3:.3f} ms ({res[B]['hbm_gbs']:.0f} GB/s)", file=sys.stderr, flush=True)
    m.close()
    return res


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "verify_c4_b1_hbm_traffic.txt")
TRAFFIC_PROFILE_B32 = os.path.join(ROOT, "profiles", "verify_c4_b32_hbm_traffic.txt")
STATS_PROFILE = os.path.join(ROOT, "profiles", "verify_c4_b1_kernel_stats.txt")
STATS_PROFILE_B32 = os.path.join(ROOT, "profiles", "verify_c4_b32_kernel_stats.txt")


def measured_traffic(key="traffic_bytes_per_launch", path=None):
    """A `key = value` line of a committed rocprofv3 summary under profiles/: HBM bytes per
    launch of a kernel class from the --pmc summaries (FETCH_SIZE and WRITE_SIZE runs of
    this script, scaled by a plain-copy calibration: the INT4 GEMV and the decode attention
    of the batch-1 verify, the many-row INT4 GEMM of the batch-32 verify), or the mean
    duration of the INT4 GEMV (batch 1) or 128-row INT4 GEMM (batch 32) launches of the
    kernel-trace summaries."""
    try:
        for line in open(path or TRAFFIC_PROFILE):
            if line.startswith(key + " "):
                return float(line.split("=")[1])
    except OSError:
        pass
    return None


def host_cpu():
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    threads = int(os.environ.get("OMP_NUM_THREADS") or avail)
    return model, os.cpu_count() or 1, avail, max(1, min(threads, avail))


def cpu_baseline(res_b1):
    """Oracle (restated reference CPU path, f32 compute) on all host cores, on a 2-layer
    slice of C4 at batch 1, extrapolated to the full model and the GPU run's round mix."""
    import refcpu as R

    model_name, nproc, avail, threads = host_cpu()
    cfg = R.make_config(vocab_size=C4["vocab_size"], hidden_dim=C4["hidden_dim"], ffn_dim=C4["ffn_dim"],
                        n_layers=2, n_heads=C4["n_heads"], n_kv_heads=C4["n_kv_heads"],
                        max_seq_len=CTX + 16, num_future_tokens=2, weight_format=R.W_INT4_G128,
                        lm_head_format=1, kv_format=R.KV_INT8)
    t0 = time.time()
    model = R.Model(cfg, seed=0, std=0.02)
    kv = model.kv(CTX + 16)
    kv.fill_synthetic(1, CTX)
    setup = time.time() - t0
    ids = np.arange(1, K_ROWS + 1, dtype=np.uint32)

    def timed(fn, reps):
        fn()
        t = time.perf_counter()
        for _ in range(reps):
            fn()
        return (time.perf_counter() - t) / reps

    t1 = timed(lambda: kv.forward_layers(ids, CTX, 1, True, threads), 3)
    t2 = timed(lambda: kv.forward_layers(ids, CTX, 2, True, threads), 3)
    per_layer = max(t2 - t1, 1e-9)
    head = max(t1 - per_layer, 0.0)
    anchor = np.random.default_rng(0).normal(0, 1, C4["hidden_dim"]).astype(np.float32)
    t_mtp = timed(lambda: model.mtp_head(0, anchor, np.array([5], np.uint32), threads), 3)
    t_verify = C4["n_layers"] * per_layer + head
    tf = res_b1["target_forwards_per_round"]
    mf = res_b1["mtp_forwards_per_round"]
    t_round = tf * t_verify + mf * t_mtp
    tok_round = res_b1["tokens_per_round"]
    return {
        "value": tok_round / t_round,
        "unit": "accepted tokens/s",
        "cores": threads,
        "kind": "port",
        "batch": 1,
        "host": {"cpu_model": model_name, "nproc": nproc, "cpus_available": avail},
        "sample": (f"CPU oracle (C restatement of the reference f32 CPU path: row-parallel online-softmax "
                   f"attention, f32 GEMV; {threads} OpenMP threads on {avail} available CPUs of '{model_name}') "
                   f"on a 2-layer slice of config 4 (INT4-dequantised f32 weights), K=4 verify rows over a "
                   f"{CTX}-token cache at batch 1: per-layer {per_layer * 1e3:.1f} ms, head {head * 1e3:.1f} ms, "
                   f"MTP head {t_mtp * 1e3:.1f} ms; extrapolated to 32 layers and the GPU run's {tf:.2f} target + "
                   f"{mf:.2f} MTP forwards and {tok_round:.2f} tokens per round.  The reference engines serve one "
                   f"request at a time, so this is also its rate at batch 32; setup {setup:.0f}s untimed"),
        "verify_ms": t_verify * 1e3,
    }


C5 = dict(vocab_size=32000, hidden_dim=2048, n_layers=24, n_heads=16, max_seq_len=4096 + 64, latent_dim=512,
          rope_dim=64, nope_dim=128, v_dim=128, n_experts=64, top_k=6, expert_dim=1408, n_shared=2)
C5_ROWS = 5  # k = 4 drafts + 1


def run_c5(args):
    """benchmark config 5 verify step: 24-layer MLA + fine-grained MoE decoder, k = 4
    (5 rows per sequence) over a 4096-token latent cache, INT4 g128 experts (MLA
    projections and router INT4 too), bf16 tied LM head."""
    import aarambh_hip as A

    cfg = A.LatConfig(**C5, expert_format=A.W_INT4_G128, attn_format=A.W_INT4_G128, lm_head_format=A.W_BF16,
                      kv_format=A.KV_F16)
    bmax = max(args.batches)
    t0 = time.time()
    m = A.HipLatModel(cfg, max_batch=bmax, max_rows=bmax * C5_ROWS)
    m.init_synthetic(seed=0, std=0.02)
    print(f"# c5 model ready in {time.time() - t0:.1f}s", file=sys.stderr, flush=True)
    rng = np.random.default_rng(0)
    res = {}
    H, D, E, NS, L = C5["hidden_dim"], C5["expert_dim"], C5["n_experts"], C5["n_shared"], C5["n_layers"]
    for B in args.batches:
        for b in range(B):
            m.kv_fill_synthetic(b, CTX, seed=1 + b)
        ids = rng.integers(1, C5["vocab_size"], (B, C5_ROWS)).astype(np.uint32)
        for _ in range(args.warmup):
            m.forward_with_cache_output(ids, [CTX] * B, want_logits=False, want_hidden=False)
        m.prof_enable(True)
        t = time.perf_counter()
        for _ in range(args.steps):
            m.forward_with_cache_output(ids, [CTX] * B, want_logits=False, want_hidden=False)
        t = (time.perf_counter() - t) / args.steps
        prof = m.prof_get()
        m.prof_enable(False)
        counts = m.expert_counts()
        used = int((counts > 0).sum())
        expert_bytes = used * 3 * (D * H // 2 + D * (H // 128) * 4)
        ffn_ms = (prof["gemv_gateup"]["ms"] + prof["gemv_down"]["ms"]) / args.steps
        res[B] = {
            "ms_per_step": t * 1e3,
            "rows_per_s": B * C5_ROWS / t,
            "experts_touched_per_layer": used / L,
            "expert_weight_bytes": expert_bytes,
            "kernels": {k: {"ms_per_step": v["ms"] / args.steps, "launches_per_step": v["launches"] / args.steps,
                            "gbs": (v["bytes"] / (v["ms"] * 1e-3) / 1e9) if v["ms"] > 0 else 0.0}
                        for k, v in prof.items() if v["launches"]},
            # expert weight bytes over the MoE block's profiled time (eager launches with events;
            # includes routing and combine, so it reads below the expert kernels' own rate)
            "moe_ffn_gbs": (prof["gemv_gateup"]["bytes"] + prof["gemv_down"]["bytes"]) / args.steps / (ffn_ms * 1e-3)
            / 1e9 if ffn_ms else 0.0,
        }
        print(f"# c5 B={B}: verify {t * 1e3:.3f} ms, {res[B]['rows_per_s']:.0f} rows/s, experts/layer "
              f"{used / L:.1f}, moe block (route + experts + combine) {res[B]['moe_ffn_gbs']:.0f} GB/s", file=sys.stderr, flush=True)
    m.close()
    return res


def c5_line(args, res):
    bmain = max(args.batches)
    r = res[bmain]
    line = {
        "metric": "config-5 verify rows/s (MLA + fine-grained MoE, INT4 experts, k=4, 4096-token latent cache)",
        "value": round(r["rows_per_s"], 1),
        "unit": "verify rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4-weight x fp16(hi+lo)-activation, f32 accumulate; fp16 latent cache",
        "data": "synthetic (random-init weights N(0,0.02^2), router N(0,1/2048), synthetic 4096-token latent cache)",
        "config": {"workload": f"C5 verify step, batch {bmain} x {C5_ROWS} rows at offset {CTX}", "batch": bmain},
        "detail": {str(b): v for b, v in res.items()},
    }
    print(json.dumps(line))


def probe_memory():
    """Two device reference figures beside the roofline peaks: the HBM rate of a plain
    device copy (read + write bytes of 256 MiB copies between four rotating buffer pairs, so
    that no launch finds its input in the 256 MB last-level cache), and the time per kernel
    of a replayed graph of 100 one-element kernels (the floor every dependent launch pays)."""
    import torch
    n = 64 << 20
    src = [torch.ones(n, dtype=torch.float32, device="cuda") for _ in range(4)]
    dst = [torch.empty_like(a) for a in src]
    for a, b in zip(src, dst):
        b.copy_(a)
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    rates = []
    for i in range(16):
        ev[0].record()
        dst[i % 4].copy_(src[i % 4])
        ev[1].record()
        torch.cuda.synchronize()
        rates.append(2 * n * 4 / (ev[0].elapsed_time(ev[1]) * 1e-3) / 1e9)
    rates = rates[4:]
    x = torch.zeros(1, device="cuda")
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        for _ in range(3):
            x.add_(1.0)
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            for _ in range(100):
                x.add_(1.0)
    torch.cuda.synchronize()
    per = []
    for _ in range(5):
        ev[0].record()
        g.replay()
        ev[1].record()
        torch.cuda.synchronize()
        per.append(ev[0].elapsed_time(ev[1]) * 1e3 / 100)
    return {"probe": "memory", "copy_bytes_read_plus_written": 2 * n * 4,
            "copy_gbs_mean": round(sum(rates) / len(rates), 1), "copy_gbs_max": round(max(rates), 1),
            "hbm_peak_gbs": HBM_PEAK_GBS, "graph_kernel_floor_us": round(min(per), 2),
            "graph_kernel_floor_us_mean": round(sum(per) / len(per), 2)}


def summarize_trace(path, title, cmd):
    """Text summary of a rocprofv3 --kernel-trace CSV (run_kernel_trace.csv) for profiles/:
    per-kernel calls / total / mean / min / max, the verify-path kernels by workgroup
    count, and the mean duration of the INT4 GEMV launches (gemv_tile_kernel<3, ...>) as
    `int4_gemv_avg_launch_us`, of the 128-row INT4 GEMM launches (gemm_kernel<3, *, 1, 2, *>
    outside the K-split mode: the 1 x 8 wave shape with two 16-row chunks per wave, which the
    C4 plan table uses above 64 rows only) as `int4_gemm128_avg_launch_us`, and of the
    INT8-cache decode attention as `attention_avg_launch_us`; bench.py quotes them beside
    its own dispatch-timed figures."""
    import csv
    rows = list(csv.DictReader(open(path)))
    col = {k.lower(): k for k in rows[0].keys()} if rows else {}
    kn, t0, t1 = col.get("kernel_name"), col.get("start_timestamp"), col.get("end_timestamp")
    wgx = col.get("grid_size_x") or col.get("grid_x")
    wsx = col.get("workgroup_size_x") or col.get("workgroup_x")
    stats, byname_wg = {}, {}
    for r in rows:
        name = r[kn].split("(")[0] if r[kn].startswith("void ") else r[kn]
        d = (int(r[t1]) - int(r[t0])) / 1000.0
        st = stats.setdefault(name, [0, 0.0, 1e30, 0.0])
        st[0] += 1
        st[1] += d
        st[2] = min(st[2], d)
        st[3] = max(st[3], d)
        if wgx and wsx:
            byname_wg.setdefault(name, set()).add(int(r[wgx]) // max(1, int(r[wsx])))
    total = sum(v[1] for v in stats.values())
    out = [f"# {title}", "# command (repository root, after `cd /tmp && export TMPDIR=/tmp`):", f"#   {cmd}",
           f"# source: {os.path.basename(path)} of that run (times in microseconds); summary by "
           f"`python3 bench.py --summarize-trace <run_kernel_trace.csv>`", "",
           f"{'kernel':74s} {'calls':>6s} {'total_ms':>9s} {'avg_us':>8s} {'min_us':>8s} {'max_us':>8s} {'pct':>6s}"]
    for name, (n, t, lo, hi) in sorted(stats.items(), key=lambda kv: -kv[1][1]):
        out.append(f"{name[:74]:74s} {n:6d} {t / 1e3:9.3f} {t / n:8.2f} {lo:8.2f} {hi:8.2f} {100 * t / total:6.2f}")
    g = [(n, t) for name, (n, t, _, _) in stats.items() if name.startswith("void aarh::gemv_tile_kernel<3,")]
    if g:
        n, t = sum(x[0] for x in g), sum(x[1] for x in g)
        out += ["", f"# all INT4 GEMV launches (gemv_tile_kernel<3, ...>): {n} dispatches, {t / 1e3:.3f} ms, mean "
                    f"{t / n:.3f} us", f"int4_gemv_avg_launch_us = {t / n:.3f}"]
    g = [(n, t) for name, (n, t, _, _) in stats.items()
         if name.startswith("void aarh::gemm_kernel<3,") and name.split("<")[1].split(",")[2:4] == [" 1", " 2"]
         and not name.rstrip().endswith("true>")]
    if g:
        n, t = sum(x[0] for x in g), sum(x[1] for x in g)
        out += ["", f"# 128-row INT4 GEMM launches (gemm_kernel<3, *, 1, 2, *, false>): {n} dispatches, {t / 1e3:.3f} ms, "
                    f"mean {t / n:.3f} us", f"int4_gemm128_avg_launch_us = {t / n:.3f}"]
    g = [(n, t) for name, (n, t, _, _) in stats.items() if name.startswith("void aarh::attn_mfma_kernel<2,")]
    if g:
        n, t = sum(x[0] for x in g), sum(x[1] for x in g)
        out += ["", f"# INT8-cache decode attention launches (attn_mfma_kernel<2, ...>): {n} dispatches, "
                    f"{t / 1e3:.3f} ms, mean {t / n:.3f} us", f"attention_avg_launch_us = {t / n:.3f}"]
    hot = [n for n in byname_wg if any(k in n for k in ("gemv_tile", "gemm_kernel", "attn", "accept", "candidates"))]
    if hot:
        out += ["", "# verify-path kernels: workgroups per launch"]
        for name in sorted(hot):
            out.append(f"{name[:74]:74s} wg {','.join(str(w) for w in sorted(byname_wg[name]))}")
    return "\n".join(out) + "\n"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=12)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--batches", type=str, default="1,8,32")
    ap.add_argument("--verify-iters", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip the config-2 and config-3 measurements")
    ap.add_argument("--workload", choices=["c4", "c5", "c2", "c3", "serve"], default="c4",
                    help="c4: the headline metric (default, with c2 / c3 / serve beside it); c5: the MLA + MoE "
                         "verify step; c2 / c3 / serve: only that measurement (profiling)")
    ap.add_argument("--c2-sampler", choices=["both", "plain", "cli"], default="both",
                    help="--workload c2: time the config's T 0.8 sampler, the reference CLI's, or both")
    ap.add_argument("--no-graphs", action="store_true",
                    help="serve workload: launch every forward directly instead of replaying captured graphs")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="run only a plain 256 MiB device copy (counter calibration for rocprof --pmc)")
    ap.add_argument("--probe-memory", action="store_true",
                    help="run only two reference measurements of the device: the HBM rate a plain device "
                         "copy reaches, and the per-kernel floor of a replayed graph")
    ap.add_argument("--summarize-trace", metavar="CSV",
                    help="print a profiles/ summary of a rocprofv3 --kernel-trace CSV and exit")
    ap.add_argument("--summary-title", default="rocprofv3 kernel statistics")
    ap.add_argument("--summary-cmd", default="")
    args = ap.parse_args()
    if args.summarize_trace:
        sys.stdout.write(summarize_trace(args.summarize_trace, args.summary_title, args.summary_cmd))
        return
    if args.probe_memory:
        print(json.dumps(probe_memory()))
        return
    if args.calibrate_copy:
        import torch
        a = torch.ones(64 << 20, dtype=torch.float32, device="cuda")
        b = torch.empty_like(a)
        for _ in range(5):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"calibration": "copy", "bytes_read": a.numel() * 4, "bytes_written": b.numel() * 4,
                          "launches": 5}))
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one MI355X; the verify path would shard by "
              "independent sequences (one engine per GPU, no collectives on the hot path) and "
              "no multi-GPU figure is produced.", file=sys.stderr)
        sys.exit(2)
    args.batches = [int(x) for x in args.batches.split(",")]
    if args.workload in ("c4", "c2") and not (args.workload == "c4" and args.no_extra):
        import torch  # torch's device runtime starts before the library's (the c2 inputs are torch tensors)
        torch.zeros(1, device="cuda")
    if args.workload == "c5":
        c5_line(args, run_c5(args))
        return
    if args.workload == "c2":
        print(json.dumps({"c2_acceptance": run_c2(args)}))
        return
    if args.workload == "c3":
        print(json.dumps({"c3_verify": {str(b): v for b, v in run_c3(args).items()}}))
        return
    if args.workload == "serve":
        print(json.dumps({"serve_continuous": run_serve(args)}))
        return
    res = run_c4(args)
    c2 = c3 = serve = c5 = None
    if not args.no_extra:
        c2 = run_c2(args)
        c3 = run_c3(args)
        serve = run_serve(args)
        c5 = run_c5(argparse.Namespace(batches=[1, 32], warmup=2, steps=5))
    bmain = max(args.batches)
    main_r = res[bmain]
    b1 = res.get(1, main_r)
    g1 = b1["int4_proj"]
    roof = {
        "kernel": "gemv_tile_kernel<INT4,4,*> (all INT4 projections of the batch-1 verify step: qkv, wo, gate/up, "
                  "down; K = 4 rows)",
        "bound": "hbm",
        "achieved": round(g1["gbs"], 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(g1["gbs"] / HBM_PEAK_GBS, 4),
        "traffic": measured_traffic(),
        "avg_launch_us": round(g1["avg_us"], 3),
        "avg_alg_bytes_per_launch": round(g1["avg_bytes"]),
    }
    # the same kernels' mean duration in the committed rocprofv3 kernel trace of this workload
    prof_us = measured_traffic("int4_gemv_avg_launch_us", STATS_PROFILE)
    if prof_us:
        gbs = g1["avg_bytes"] / (prof_us * 1e-6) / 1e9
        roof["profile"] = {"file": os.path.relpath(STATS_PROFILE, ROOT), "avg_launch_us": prof_us,
                           "achieved": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}
    a1 = b1["attention"]
    roof_att = {
        "kernel": "attn_mfma_kernel<INT8> (decode attention of the batch-1 verify step, 4096-token INT8 cache)",
        "bound": "hbm", "achieved": round(a1["gbs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
        "frac": round(a1["gbs"] / HBM_PEAK_GBS, 4), "traffic": measured_traffic("attention_traffic_bytes_per_launch"),
        "avg_launch_us": round(a1["avg_us"], 3),
        "avg_alg_bytes_per_launch": round(a1["alg_bytes_per_step"] / C4["n_layers"]),
    }
    def att_profile(a, path):
        """The same launches' mean duration in a committed rocprofv3 kernel trace summary."""
        us = measured_traffic("attention_avg_launch_us", path)
        if not us:
            return None
        gbs = a["alg_bytes_per_step"] / C4["n_layers"] / (us * 1e-6) / 1e9
        return {"file": os.path.relpath(path, ROOT), "avg_launch_us": us, "achieved": round(gbs, 1),
                "frac": round(gbs / HBM_PEAK_GBS, 4)}
    prof = att_profile(a1, STATS_PROFILE)
    if prof:
        roof_att["profile"] = prof
    roof_att32 = None
    if 32 in res:
        a32 = res[32]["attention"]
        roof_att32 = {
            "kernel": "attn_mfma_kernel<INT8> (decode attention of the batch-32 verify step, 4096-token INT8 cache)",
            "bound": "hbm", "achieved": round(a32["gbs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(a32["gbs"] / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic("attention_traffic_bytes_per_launch", TRAFFIC_PROFILE_B32),
            "avg_launch_us": round(a32["avg_us"], 3),
            "avg_alg_bytes_per_launch": round(a32["alg_bytes_per_step"] / C4["n_layers"]),
        }
        prof = att_profile(a32, STATS_PROFILE_B32)
        if prof:
            roof_att32["profile"] = prof
    roof_gemm = None
    if 32 in res:
        gm = res[32]["int4_proj"]
        roof_gemm = {
            "kernel": "gemm_kernel<INT4,*> (INT4 projections of the batch-32 verify step, M = 128 rows; useful "
                      "FLOPs 2*M*N*K, the fp16 hi + lo activation split issues twice as many)",
            "bound": "mfma", "achieved": round(gm["useful_tflops"], 1), "peak": MFMA_F16_PEAK_TFLOPS,
            "unit": "TFLOP/s", "frac": round(gm["useful_tflops"] / MFMA_F16_PEAK_TFLOPS, 4),
            "traffic": measured_traffic("gemm_traffic_bytes_per_launch", TRAFFIC_PROFILE_B32),
            "avg_launch_us": round(gm["avg_us"], 3),
        }
        # the same launches' mean duration in the committed rocprofv3 kernel trace
        prof_us = measured_traffic("int4_gemm128_avg_launch_us", STATS_PROFILE_B32)
        if prof_us and gm["avg_us"]:
            tf = gm["useful_tflops"] * gm["avg_us"] / prof_us
            roof_gemm["profile"] = {"file": os.path.relpath(STATS_PROFILE_B32, ROOT), "avg_launch_us": prof_us,
                                    "achieved": round(tf, 1), "frac": round(tf / MFMA_F16_PEAK_TFLOPS, 4)}
    cpu = None
    if not args.no_cpu and 1 in res:
        try:
            cpu = cpu_baseline(res[1])
        except Exception as exc:  # the CPU leg must not hide the GPU result
            cpu = {"error": str(exc)}
    line = {
        "metric": METRIC,
        "value": round(main_r["tokens_per_s"], 2),
        "unit": "accepted tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(main_r["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4-weight x fp16(hi+lo)-activation, f32 accumulate",
        "data": "synthetic (random-init weights N(0,0.02^2), synthetic 4096-token INT8 KV, greedy MTP)",
        "config": {"workload": f"C4 INT4 g128 MTP k=3 verify rounds, batch {bmain} (batches "
                               f"{','.join(str(b) for b in args.batches)} beside), 4096-token INT8 KV",
                   "batch": bmain, "verify_rows_per_seq": K_ROWS, "context": CTX},
        "per_batch": {str(b): {k: r[k] for k in ("tokens_per_s", "ms_per_step", "acceptance_rate",
                                                 "tokens_per_round")} for b, r in res.items()},
        "per_batch_sampled_cli": {str(b): r["sampled_cli"] for b, r in res.items()},
        "verify_step": {str(b): {k: r["verify"][k] for k in ("ms_wall", "ms_kernels", "alg_bytes", "hbm_gbs",
                                                               "hbm_frac")} for b, r in res.items()},
        "roofline": roof,
        "roofline_attention": roof_att,
        "roofline_attention_b32": roof_att32,
        "roofline_gemm": roof_gemm,
        "c2_acceptance": c2,
        "c3_verify": {str(b): {k: v[k] for k in ("ms_wall", "alg_bytes", "hbm_gbs", "hbm_frac")}
                      for b, v in c3.items()} if c3 else None,
        "serve_continuous": serve,
        "c5_verify": {str(b): {k: v[k] for k in ("ms_per_step", "rows_per_s", "experts_touched_per_layer", "moe_ffn_gbs")}
                      for b, v in c5.items()} if c5 else None,
        "cpu_baseline": cpu,
        "detail": {"c4": {str(b): r for b, r in res.items()},
                   "c3": {str(b): v for b, v in c3.items()} if c3 else None},
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
