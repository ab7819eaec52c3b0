"""Decode-GEMV benchmark for the MI355X k-quant path (BASELINE metric:
"Q4_K GEMV HBM GB/s (% of peak) + batch-1 decode tok/s, Qwen3-8B shapes").

One step = the quantized-projection work of one batch-1 Qwen3-8B decode token:
for each of 36 layers, RMSNorm-fused q/k/v (Q4_K 4096->4096/1024/1024), o
(Q4_K 4096->4096), RMSNorm-fused gate/up (Q4_K 4096->12288) and down (Q5_K
12288->4096), then the RMSNorm-fused Q6_K lm_head (4096->151936). Every layer
has its own synthetic weights (4.64 GB per step, far beyond the 256 MB
Infinity Cache), resident in HBM before timing starts. Attention, SwiGLU and
residual kernels are not part of this step (the activations are synthetic).

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Prints one JSON line. `value` is achieved algorithmic GB/s over the timed
steps (weights + f32 activations in + f32 outputs, each once per launch).
"""
from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0
PEAK_BF16_TFLOPS = 2500.0  # dense bf16 / f16 MFMA
HIDDEN, FFN, Q_OUT, KV_OUT, VOCAB = 4096, 12288, 4096, 1024, 151936
EPS = 1e-6
METRIC = "Q4_K GEMV HBM GB/s (% of peak) + batch-1 decode tok/s, Qwen3-8B shapes"

# (name, value type, K, N, norm group) per layer, in decode order (decode.rs:544-696).
LAYER = [
    ("q", 12, HIDDEN, Q_OUT, "attn"),
    ("k", 12, HIDDEN, KV_OUT, "attn"),
    ("v", 12, HIDDEN, KV_OUT, "attn"),
    ("o", 12, Q_OUT, HIDDEN, None),
    ("gate", 12, HIDDEN, FFN, "ffn"),
    ("up", 12, HIDDEN, FFN, "ffn"),
    ("down", 13, FFN, HIDDEN, None),
]
BLOCK_BYTES = {12: 144, 13: 176, 14: 210}


def launch_bytes(t, k, n):
    return k // 256 * n * BLOCK_BYTES[t] + 4 * k + 4 * n


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def build_model(E, synth, torch, layers, seed):
    gen = torch.Generator(device="cuda:0")
    gen.manual_seed(seed)
    dev = torch.device("cuda:0")
    weights = []
    for li in range(layers):
        lw = {}
        for name, t, k, n, _ in LAYER:
            lw[name] = (t, k, n, synth.kquant_torch(t, k, n, gen, dev))
        lw["attn_gamma"] = 1.0 + 0.02 * torch.randn(HIDDEN, device=dev, generator=gen)
        lw["ffn_gamma"] = 1.0 + 0.02 * torch.randn(HIDDEN, device=dev, generator=gen)
        weights.append(lw)
    head = (14, HIDDEN, VOCAB, synth.kquant_torch(14, HIDDEN, VOCAB, gen, dev))
    out_gamma = 1.0 + 0.02 * torch.randn(HIDDEN, device=dev, generator=gen)
    acts = {
        "hidden": torch.randn(HIDDEN, device=dev, generator=gen),
        "attn_out": torch.randn(Q_OUT, device=dev, generator=gen),
        "ffn_act": torch.randn(FFN, device=dev, generator=gen),
    }
    return weights, head, out_gamma, acts


class DecodeGemvStep:
    """Issues one step's launches through the C ABI on ctx's stream."""

    def __init__(self, E, torch, ctx, weights, head, out_gamma, acts, mode=0):
        self.store = E.AmdWeightStore(ctx)
        self.kern = {t: E.QwenGemvKernel.from_value_type(ctx, t) for t in (12, 13, 14)}
        self.set_mode(mode)
        self.layers = []
        for li, lw in enumerate(weights):
            entry = {}
            for name, t, k, n, norm in LAYER:
                key = f"blk.{li}.{name}"
                self.store.materialize_quantized(key, [k, n], t, lw[name][3])
                entry[name] = (self.store.quantized_tensor(key), t, k, n, norm)
            entry["attn_gamma"] = lw["attn_gamma"]
            entry["ffn_gamma"] = lw["ffn_gamma"]
            self.layers.append(entry)
        self.store.materialize_quantized("output", [HIDDEN, VOCAB], 14, head[3])
        self.head = self.store.quantized_tensor("output")
        self.out_gamma = out_gamma
        self.acts = acts
        self.outs = {name: torch.empty(n, device="cuda:0") for name, _, _, n, _ in LAYER}
        self.logits = torch.empty(VOCAB, device="cuda:0")
        # Algorithmic bytes per launch: encoded weights + f32 input once + f32 outputs.
        qkv = sum(launch_bytes(12, HIDDEN, n) - 4 * HIDDEN for n in (Q_OUT, KV_OUT, KV_OUT)) + 4 * HIDDEN
        gate_up = 2 * (launch_bytes(12, HIDDEN, FFN) - 4 * HIDDEN) + 4 * HIDDEN
        per_layer = qkv + launch_bytes(12, Q_OUT, HIDDEN) + gate_up + launch_bytes(13, FFN, HIDDEN)
        self.bytes_per_step = per_layer * len(weights) + launch_bytes(14, HIDDEN, VOCAB)

    def set_mode(self, mode):
        for k in self.kern.values():
            k.set_mode(mode)

    def layer(self, entry):
        # q/k/v share the attention-normed input and gate/up the FFN-normed
        # input: each group is one launch with RMSNorm fused into its prologue.
        k4 = self.kern[12]
        k4.execute_group([entry[n][0] for n in ("q", "k", "v")], self.acts["hidden"],
                         [self.outs[n] for n in ("q", "k", "v")], 1, entry["attn_gamma"], EPS)
        k4.execute_warp(entry["o"][0], self.acts["attn_out"], self.outs["o"])
        k4.execute_group([entry[n][0] for n in ("gate", "up")], self.acts["hidden"],
                         [self.outs[n] for n in ("gate", "up")], 1, entry["ffn_gamma"], EPS)
        self.kern[13].execute_warp(entry["down"][0], self.acts["ffn_act"], self.outs["down"])

    def run(self):
        for entry in self.layers:
            self.layer(entry)
        self.kern[14].execute_rms_norm(self.head, self.acts["hidden"], self.out_gamma, EPS, self.logits, 1)

    def run_gate_up(self):
        for entry in self.layers:
            self.kern[12].execute_group([entry[n][0] for n in ("gate", "up")], self.acts["hidden"],
                                        [self.outs[n] for n in ("gate", "up")], 1, entry["ffn_gamma"], EPS)


def capture(torch, stream, fn):
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        fn()
    return g


def _time_median(fn, budget_s, max_runs=20, min_runs=5, warmup=3):
    """Median and minimum seconds of fn() after `warmup` runs: up to max_runs
    runs within budget_s (at least min_runs)."""
    for _ in range(warmup):
        fn()
    samples = []
    t_end = time.perf_counter() + budget_s
    while len(samples) < max_runs and (time.perf_counter() < t_end or len(samples) < min_runs):
        t0 = time.perf_counter()
        fn()
        samples.append(time.perf_counter() - t0)
    samples.sort()
    return samples[len(samples) // 2], samples[0], len(samples)


def cpu_baseline(seconds_budget=12.0):
    """The reference's CPU path restated in C (oracle/kquant_oracle.c, built
    -O2 -ffp-contract=off): dequantize_block per super-block, then the
    sequential f32 dot (crates/gguf/src/lib.rs:520-661,
    crates/nvidia/src/qwen_reference.rs:31-40). Primary input BASELINE
    config 0 (one 4096x4096 Q4_K matvec) on 1 thread, as the reference runs
    it; also on every host core (rows split across threads) and the config-1
    layer (RMSNorm + the seven projections) on 1 thread."""
    import numpy as np

    from engine_amd import synth
    from oracle import kquant_oracle as O

    nproc = os.cpu_count() or 1
    threads_all = min(16, nproc)  # the GPU box grants 16 host threads per GPU
    k0 = n0 = 4096
    enc0 = synth.kquant_numpy(12, k0, n0, seed=500)
    x0 = synth.activations_numpy(k0, 1, seed=501)[0]
    bytes0 = launch_bytes(12, k0, n0)
    med1, min1, runs1 = _time_median(lambda: O.quant_gemv(12, enc0, k0, n0, x0, threads=1), seconds_budget / 3)
    med_all, _, runs_all = _time_median(lambda: O.quant_gemv(12, enc0, k0, n0, x0, threads=threads_all),
                                        seconds_budget / 6)

    mats = [(t, k, n, synth.kquant_numpy(t, k, n, seed=510 + i)) for i, (_, t, k, n, _) in enumerate(LAYER)]
    x = {k: synth.activations_numpy(k, 1, seed=k)[0] for k in (HIDDEN, FFN)}
    gamma = synth.gamma_numpy(HIDDEN, seed=9)
    layer_bytes = sum(launch_bytes(t, k, n) for t, k, n, _ in mats)

    def one_layer():
        normed = O.rms_norm_raw(x[HIDDEN], gamma, EPS)
        for t, k, n, enc in mats:
            O.quant_gemv(t, enc, k, n, normed if k == HIDDEN else x[FFN], threads=1)

    med_layer, _, runs_layer = _time_median(one_layer, seconds_budget / 2, max_runs=20, min_runs=3, warmup=1)
    return {
        "value": round(bytes0 / med1 / 1e9, 4),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": (f"BASELINE config 0: Q4_K 4096x4096 matvec ({bytes0} algorithmic bytes, "
                   f"{2 * k0 * n0} flop), oracle/kquant_oracle.c -O2 -ffp-contract=off, 1 thread, "
                   f"median of {runs1} runs after 3 warm-ups ({med1 * 1e3:.2f} ms; min {min1 * 1e3:.2f} ms)"),
        "gflop_s": round(2 * k0 * n0 / med1 / 1e9, 3),
        "all_cores": {"value": round(bytes0 / med_all / 1e9, 3), "unit": "GB/s", "cores": threads_all,
                      "ms": round(med_all * 1e3, 3), "runs": runs_all},
        "layer_1_thread": {"value": round(layer_bytes / med_layer / 1e9, 4), "unit": "GB/s", "bytes": layer_bytes,
                           "ms": round(med_layer * 1e3, 2), "runs": runs_layer,
                           "sample": "BASELINE config 1: RMSNorm + q,k,v,o,gate,up Q4_K + down Q5_K"},
        "nproc": nproc,
        "host_cpu": _cpu_model(),
    }


PEAK_MFMA_F16_TFLOPS = 2500.0  # MI355X dense f16/bf16
# GEMV arithmetic (include/ribn_amd.h RIBN_AMD_GEMV_*)
GEMV_MODES = {"warp": 0, "fixed16": 1}
KV_BYTES_PER_TOKEN = 36 * 8 * 128 * 2 * 2  # f16 K and V of every layer: 147,456 B


def build_decoder(E, synth, torch, ctx, step, out_gamma, layers, seed, members):
    """The full Qwen3-8B-shaped decoder, random-init and
    seeded: its own weights of the step's shapes (Q4_K q/k/v/o/gate/up, Q5_K
    down, Q6_K lm_head, a Q4_K token_embd table), drawn centered (zero-mean
    weights, so greedy decoding does not settle on one token; the same bytes
    and kernels as the GEMV chain), the step's RMSNorm gammas and per-head q/k
    norms. Built once and cached on the step."""
    cached = getattr(step, "decoder_weights", None)
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed + 1)
    if cached is None:
        store = E.AmdWeightStore(ctx)
        store.materialize_quantized("token_embd", [HIDDEN, VOCAB], 12,
                                    synth.kquant_torch(12, HIDDEN, VOCAB, gen, dev, centered=True))
        store.materialize_quantized("output", [HIDDEN, VOCAB], 14,
                                    synth.kquant_torch(14, HIDDEN, VOCAB, gen, dev, centered=True))
        per_layer = []
        for li in range(len(step.layers)):
            lw = {}
            for name, t, k, n, _ in LAYER:
                store.materialize_quantized(f"blk.{li}.{name}", [k, n], t,
                                            synth.kquant_torch(t, k, n, gen, dev, centered=True))
                lw[name] = store.quantized_tensor(f"blk.{li}.{name}")
            per_layer.append(lw)
        cached = step.decoder_weights = (store, per_layer)
    store, per_layer = cached
    names = {"q": "attn_q", "k": "attn_k", "v": "attn_v", "o": "attn_output", "gate": "ffn_gate",
             "up": "ffn_up", "down": "ffn_down"}
    plan = []
    for entry, lwq in zip(step.layers[:layers], per_layer):
        lw = {names[n]: lwq[n] for n in names}
        lw["attn_norm"] = entry["attn_gamma"]
        lw["ffn_norm"] = entry["ffn_gamma"]
        lw["attn_q_norm"] = 1.0 + 0.02 * torch.randn(128, device=dev, generator=gen)
        lw["attn_k_norm"] = 1.0 + 0.02 * torch.randn(128, device=dev, generator=gen)
        plan.append(lw)
    cfg = E.AmdQwen3Config(layers=layers)
    dec = E.AmdQwen3Decode(ctx, cfg, store.quantized_tensor("token_embd"), store.quantized_tensor("output"),
                           out_gamma, plan, members)
    dec.set_gemv_mode(GEMV_MODES[getattr(build_decoder, "mode", "warp")])
    return dec, cfg


def time_model_decode(E, dec, cfg, ctx, members, context, gen_tokens, seed, prompt_chunk=2048):
    """Prefills `context` prompt tokens per member, then times `gen_tokens`
    greedy steps of the graph-replayed generation loop (wall clock, which
    includes the step's host work). Member m's prompt depends on the seed and
    m only, so member 0 has the same prompt at every batch size. The first
    context - 1 tokens of each prompt run through prefill_prompt (the prefill
    matmul, chunks of `prompt_chunk`; timed with the workspace already
    reserved, `prompt_tok_s` = prompt tokens per second over all members),
    or with prompt_chunk = 0 as serial single-token steps (the reference's
    prefill_step). Returns the result line, the generated tokens and member
    0's last logits."""
    import numpy as np
    rng = np.random.default_rng(seed)
    # rows are drawn in order, so member m's prompt is the same at every batch size
    prompts = rng.integers(0, VOCAB, size=(max(8, members), context))[:members]
    caches = [E.AmdKvCache(ctx, cfg, context + gen_tokens) for _ in range(members)]
    if prompt_chunk:
        dec.reserve_prompt(prompt_chunk)
    ctx.synchronize()
    t0 = time.perf_counter()
    if prompt_chunk:
        for m in range(members):
            dec.prefill_prompt(caches[m], prompts[m, :context - 1], 0, prompt_chunk)
    else:
        for p in range(context - 1):
            if members == 1:
                dec.prefill_step(caches[0], int(prompts[0, p]), p)
            else:
                dec.decode_step_batch(caches, prompts[:, p], [p] * members)
    ctx.synchronize()
    prefill_s = time.perf_counter() - t0
    last = prompts[:, context - 1]
    start = [context - 1] * members
    dec.generate(caches, last, start, 1)  # captures the loop's graph; rewrites slot context-1 identically
    t0 = time.perf_counter()
    out = dec.generate(caches, last, start, gen_tokens)
    dt = time.perf_counter() - t0
    kv_read = sum((context + s) * KV_BYTES_PER_TOKEN * cfg.layers // 36 for s in range(gen_tokens)) / gen_tokens
    line = {"members": members, "context": context, "generated": gen_tokens,
            "tok_s": round(members * gen_tokens / dt, 1), "ms_per_step": round(dt * 1e3 / gen_tokens, 4),
            "prefill_s": round(prefill_s, 3), "prompt_chunk": prompt_chunk,
            "prompt_tok_s": round(members * (context - 1) / prefill_s, 1), "kv_bytes_per_step": int(kv_read * members),
            "distinct_tokens": int(len(set(out.reshape(-1).tolist())))}
    return line, out, dec.copy_logits(0)


def model_decode_results(E, synth, torch, ctx, step, out_gamma, args):
    """Batch 1, then batch 8 whose member 0 has batch 1's prompt. In the f32
    GEMV mode member 0's tokens and last logits equal batch 1's bit for bit
    (`b8_member0_bitwise_equal_b1`): a check on the timed run itself, beside
    `distinct_tokens` (the centered random weights give varied greedy tokens).
    Then batch 16, whose projections run on the f32-faithful matrix-core GEMV
    (weights read once for the batch; rows agree with batch 1 to f32 rounding,
    not bit for bit)."""
    import numpy as np
    dec, cfg = build_decoder(E, synth, torch, ctx, step, out_gamma, args.layers, args.seed, 16)
    res, runs = {}, {}
    for members in (1, 8, 16):
        r, toks, logits = time_model_decode(E, dec, cfg, ctx, members, args.context, args.gen_tokens, args.seed,
                                            args.prompt_chunk)
        log(f"bench model: batch {members}: {r['tok_s']} tok/s ({r['ms_per_step']} ms/step, "
            f"prompt {r['prompt_tok_s']} tok/s in {r['prefill_s']} s)")
        res[members] = r
        runs[members] = (toks[0], logits)
    res["b8_member0_bitwise_equal_b1"] = bool(np.array_equal(runs[1][0], runs[8][0]) and
                                              np.array_equal(runs[1][1].view(np.uint32),
                                                             runs[8][1].view(np.uint32)))
    log(f"bench model: batch-8 member 0 bit-identical to batch 1: {res['b8_member0_bitwise_equal_b1']}")
    dec.close()
    return res


def _graph_time_us(torch, stream, fn, reps):
    """Mean microseconds of fn() replayed as a HIP graph `reps` times on `stream`."""
    with torch.cuda.stream(stream):
        fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        fn()
    with torch.cuda.stream(stream):
        g.replay()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(reps):
            g.replay()
        b.record(stream)
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e3 / reps


def batched_ffn_times(E, synth, torch, args, ms=(1, 4, 8, 16, 64), compare=True):
    """the Qwen3-8B FFN (gate/up Q4_K 4096->12288, down Q5_K 12288->4096)
    for M tokens with f32 activations ~N(0,1), through the decode step's batched GEMV entry
    points (gate/up as one grouped launch). The default f32 arithmetic (GEMV_WARP) runs the f32
    wave GEMV up to 8 members (weights read once per launch group, every row bit-identical to
    the single call) and the f32-faithful matrix-core GEMV from 9 to 64 members (Q4_K / Q5_K:
    quants times group scale exact in f16 against activations in two f16 pieces with a per-block
    power-of-two scale, f16 MFMA with f32 accumulation; weights read once for the batch).
    For comparison: the opt-in block fixed-point mode at M <= 16 and the f16 prefill matmul at
    M = 64."""
    dev = torch.device("cuda:0")
    stream = torch.cuda.Stream()
    ctx = E.AmdContext(0, stream=stream)
    ctx.reserve_prefill(64, FFN, FFN)
    store = E.AmdWeightStore(ctx)
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    layers = []
    n_layers = 8  # 730 MB of distinct weights, ~3x the 256 MB Infinity Cache
    for i in range(n_layers):
        for name, t, k, n in (("gate", 12, HIDDEN, FFN), ("up", 12, HIDDEN, FFN), ("down", 13, FFN, HIDDEN)):
            store.materialize_quantized(f"{name}{i}", [k, n], t, synth.kquant_torch(t, k, n, gen, dev))
        layers.append({nm: store.quantized_tensor(f"{nm}{i}") for nm in ("gate", "up", "down")})
    k4, k5 = E.AmdQ4KGemv.from_context(ctx), E.AmdQ5KGemv.from_context(ctx)
    wbytes = 2 * (FFN * HIDDEN // 256 * 144) + HIDDEN * FFN // 256 * 176
    per_m = {}
    for m in ms:
        x = torch.randn(m, HIDDEN, device=dev, generator=gen)
        h = torch.randn(m, FFN, device=dev, generator=gen)
        g, u, d = (torch.empty(m * n, device=dev) for n in (FFN, FFN, HIDDEN))

        def gemv_ffn():
            for ly in layers:
                k4.execute_group([ly["gate"], ly["up"]], x, [g, u], m)
                k5.execute_warp_batch(ly["down"], h, d, m)
        runs = [("warp", "f32 wave GEMV, weights read once per launch group of up to 8 members (down's K = 12288 "
                         "split by slice from 3 members, with an ordered slice reduction)" if m <= 8 else
                 "f32-faithful matrix-core GEMV (quants x group scale exact in f16, x in two f16 pieces, f16 MFMA "
                 "with f32 accumulation, f32 block epilogue), weights read once for the batch", gemv_ffn)]
        if compare and m <= 16:
            runs.append(("fixed16", "block fixed-point " + ("wave GEMV" if m < 4 else
                         "wave GEMV gate/up, matrix-core GEMV down" if m < 5 else "matrix-core GEMV") +
                         ", weights read once per launch", gemv_ffn))
        elif compare:
            def prefill_ffn():
                for ly in layers:
                    k4.gemm_prefill(ly["gate"], x, g, m)
                    k4.gemm_prefill(ly["up"], x, u, m)
                    k5.gemm_prefill(ly["down"], h, d, m)
            runs.append(("f16-mfma", "prefill matmul (activations rounded to f16, f16 MFMA, f32 accumulation)",
                         prefill_ffn))
        per_m[m] = {}
        for mode, path, fn in runs:
            for kern in (k4, k5):
                kern.set_mode(GEMV_MODES.get(mode, 0))
            us = _graph_time_us(torch, stream, fn, max(2, args.steps // 10)) / n_layers
            flops = 2.0 * m * 3 * FFN * HIDDEN
            per_m[m][mode] = {"us_per_ffn": round(us, 2), "tokens_per_s": round(m * 1e6 / us, 1),
                              "weight_GBps": round(wbytes / us / 1e3, 1), "hbm_frac": round(wbytes / us / 1e3 / PEAK_HBM_GBS, 4),
                              "tflops": round(flops / us / 1e6, 2), "path": path}
            if mode == "warp" and m > 8:
                # executed on the matrix cores as two f16 products (the activation's two pieces) per f32 one
                per_m[m][mode]["f16_mfma_frac"] = round(2 * flops / us / 1e6 / PEAK_BF16_TFLOPS, 4)
            log(f"bench batched: M={m} {mode}: {us:.2f} us per FFN ({path})")
        for kern in (k4, k5):
            kern.set_mode(0)
    return per_m, wbytes, n_layers


def bench_batched(E, synth, torch, args):
    """BASELINE config 2 as its own bench line: every M in f32 mode, with the opt-in comparisons."""
    per_m, wbytes, n_layers = batched_ffn_times(E, synth, torch, args)
    top = per_m[64]["warp"]
    return {
        "metric": "batched decode FFN throughput (BASELINE config 2), tokens/s at M=64, f32 activations",
        "value": top["tokens_per_s"], "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(top["us_per_ffn"] / 1e3, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32 (M>=9 on f16 MFMA with exact two-piece activations, f32 accumulation); per_m also holds "
                 "i8dot4 / i8-mfma (fixed16) for M<=16 and f16-mfma at M=64",
        "data": "synthetic",
        "config": {"workload": "qwen3-8b-ffn-batched", "ffn_weight_bytes": wbytes, "layers_cycled": n_layers,
                   "per_m": per_m},
        "roofline": {"bound": "hbm", "achieved": per_m[1]["warp"]["weight_GBps"], "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(per_m[1]["warp"]["weight_GBps"] / PEAK_HBM_GBS, 4),
                     "traffic": None, "kernel": "M=1 FFN (gate/up group + down), f32 wave GEMV"},
        "cpu_baseline": None,
    }


def bench_q8_1(E, synth, torch, args):
    """The Q8_1 integer-dot path (the reference's GemvMode::IntegerDot, decode.rs:1341-1478):
    per projection, pack the activations into Q8_1 blocks, then the integer-dot
    GEMV, over the seven Qwen3-8B layer projections (Q4_K q/k/v/o/gate/up, Q5_K
    down) of 8 distinct layers, graph-replayed, at batch 1 and 8. Lossy by
    design (8-bit activations); reported beside the default f32-activation path."""
    dev = torch.device("cuda:0")
    stream = torch.cuda.Stream()
    ctx = E.AmdContext(0, stream=stream)
    store = E.AmdWeightStore(ctx)
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    n_layers = 8
    layers = []
    for i in range(n_layers):
        ly = {}
        for name, t, k, n, _ in LAYER:
            store.materialize_quantized(f"{name}{i}", [k, n], t, synth.kquant_torch(t, k, n, gen, dev))
            ly[name] = (store.quantized_tensor(f"{name}{i}"), t, k, n)
        layers.append(ly)
    quant = E.AmdQ8_1Quantizer(ctx)
    gemv = {12: E.AmdQ4KQ8_1Gemv(ctx), 13: E.AmdQ5KQ8_1Gemv(ctx)}
    wbytes = sum(launch_bytes(t, k, n) - 4 * k - 4 * n for _, t, k, n, _ in LAYER)
    per_m = {}
    for m in (1, 8):
        xs = {k: torch.randn(m * k, device=dev, generator=gen) for k in (HIDDEN, FFN)}
        packed = {k: torch.empty(m * k // 32 * 9, dtype=torch.int32, device=dev) for k in (HIDDEN, FFN)}
        outs = {n: torch.empty(m * n, device=dev) for n in (Q_OUT, KV_OUT, FFN, HIDDEN)}

        def fn():
            for ly in layers:
                for name, _, k, n, _ in LAYER:
                    w, t, k, n = ly[name]
                    quant.execute(xs[k], packed[k])
                    if m == 1:
                        gemv[t].execute(w, packed[k], outs[n])
                    else:
                        gemv[t].execute_batch(w, packed[k], outs[n], m)

        us = _graph_time_us(torch, stream, fn, max(2, args.steps // 10)) / n_layers
        per_m[m] = {"us_per_layer": round(us, 2), "weight_GBps": round(wbytes / us / 1e3, 1),
                    "tokens_per_s_36_layers": round(m * 1e6 / (36 * us), 1)}
        log(f"bench q8_1: M={m} {us:.2f} us per layer (7 packs + 7 integer-dot GEMVs), "
            f"{wbytes / us / 1e3:.0f} GB/s of weights")
    top = per_m[1]
    return {
        "metric": "Q8_1 integer-dot decode projections, weight GB/s at batch 1",
        "value": top["weight_GBps"], "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(top["us_per_layer"] / 1e3, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "i8dot4 (q8_1 activations)", "data": "synthetic",
        "config": {"workload": "qwen3-8b-layer-q8_1", "layer_weight_bytes": wbytes, "layers_cycled": n_layers,
                   "per_m": per_m},
        "roofline": {"bound": "hbm", "achieved": top["weight_GBps"], "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(top["weight_GBps"] / PEAK_HBM_GBS, 4), "traffic": None,
                     "kernel": "q8_1_gemv_kernel + quantize_q8_1_kernel over one layer"},
        "cpu_baseline": None,
    }


# The reference's own GEMV figures (`crates/nvidia/examples/int_dot_bench.rs`, shapes at :24,
# weight bytes / median host-timed launch + synchronize at :493-525), RTX 4090, weight GB/s,
# `benchmarks/qwen-prefill-qualification.md:515-523` ("after" columns): (batch 1, batch 8).
PUBLISHED_SHAPES = ((5120, 5120), (5120, 17408), (17408, 5120))
PUBLISHED_RTX4090 = {
    12: ((1027.4, 276.1), (1454.1, 433.3), (1353.8, 296.2)),
    13: ((975.0, 323.3), (1303.2, 504.1), (1178.5, 351.7)),
    14: ((1157.6, 403.9), (1537.7, 597.1), (1417.0, 418.4)),
}


def bench_published(E, synth, torch, args):
    """The reference's published GEMV shapes (Qwen3.x-27B: K x N = 5120x5120, 5120x17408,
    17408x5120) for Q4_K / Q5_K / Q6_K, batch 1 (execute_warp) and 8 members
    (execute_warp_batch), weight GB/s = encoded weight bytes / time per launch, three ways:
    - host: the reference's method (one matrix, launch + synchronize timed on the host,
      median of --steps iterations); the matrix stays cache-resident, like the RTX 4090
      figures it sits beside (every one of these matrices fits that card's 72 MB L2);
    - resident: the same matrix, back-to-back launches replayed as a HIP graph, device time
      per launch (the matrix sits in the 256 MB Infinity Cache);
    - hbm: launches rotate over distinct copies of the matrix totalling at least 1 GB, so
      every launch streams its weights from HBM (the roofline figure)."""
    import math
    import statistics

    dev = torch.device("cuda:0")
    stream = torch.cuda.Stream()
    ctx = E.AmdContext(0, stream=stream)
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    iters = max(20, args.steps)
    rows_out = []
    for t in (12, 13, 14):
        kern = E.QwenGemvKernel.from_value_type(ctx, t)
        for si, (k, n) in enumerate(PUBLISHED_SHAPES):
            wbytes = n * (k // 256) * BLOCK_BYTES[t]
            base = synth.kquant_torch(t, k, n, gen, dev)
            copies = max(2, math.ceil(1.0e9 / wbytes))
            store = E.AmdWeightStore(ctx)
            tensors = [base] + [base.clone() for _ in range(copies - 1)]
            ws = []
            for ci, enc in enumerate(tensors):
                store.materialize_quantized(f"w{ci}", [k, n], t, enc)
                ws.append(store.quantized_tensor(f"w{ci}"))
            for members in (1, 8):
                x = torch.randn(members * k, device=dev, generator=gen)
                y = torch.empty(members * n, device=dev)

                def one(w):
                    if members == 1:
                        kern.execute_warp(w, x, y)
                    else:
                        kern.execute_warp_batch(w, x, y, members)

                with torch.cuda.stream(stream):
                    for _ in range(5):
                        one(ws[0])
                torch.cuda.synchronize()
                host = []
                for _ in range(iters):
                    t0 = time.perf_counter()
                    with torch.cuda.stream(stream):
                        one(ws[0])
                    stream.synchronize()
                    host.append(time.perf_counter() - t0)
                host_us = statistics.median(host) * 1e6
                reps = max(2, iters // 10)
                resident_us = _graph_time_us(torch, stream, lambda: [one(ws[0]) for _ in range(32)], reps) / 32
                hbm_us = _graph_time_us(torch, stream, lambda: [one(w) for w in ws], reps) / len(ws)
                pub = PUBLISHED_RTX4090[t][si][0 if members == 1 else 1]
                row = {"type": {12: "Q4_K", 13: "Q5_K", 14: "Q6_K"}[t], "k": k, "n": n, "members": members,
                       "weight_bytes": wbytes, "copies_rotated": len(ws),
                       "host_us": round(host_us, 2), "host_GBps": round(wbytes / host_us / 1e3, 1),
                       "resident_us": round(resident_us, 2), "resident_GBps": round(wbytes / resident_us / 1e3, 1),
                       "hbm_us": round(hbm_us, 2), "hbm_GBps": round(wbytes / hbm_us / 1e3, 1),
                       "hbm_frac": round(wbytes / hbm_us / 1e3 / PEAK_HBM_GBS, 4),
                       "rtx4090_published_GBps": pub}
                rows_out.append(row)
                log(f"bench published: {row['type']} {k}x{n} M={members}: host {row['host_GBps']} GB/s, "
                    f"resident {row['resident_GBps']}, hbm {row['hbm_GBps']} ({row['hbm_frac']:.1%}); "
                    f"RTX 4090 published {pub}")
            for w in ws:
                w.close()
            del ws, tensors, base, store
            torch.cuda.synchronize()
            torch.cuda.empty_cache()
        kern.close()
    q4 = [r for r in rows_out if r["type"] == "Q4_K" and r["members"] == 1]
    hbm = sum(r["weight_bytes"] for r in q4) / sum(r["hbm_us"] for r in q4) / 1e3
    return {
        "metric": "Q4_K warp GEMV weight GB/s at the reference's published shapes, batch 1, HBM-streamed",
        "value": round(hbm, 1), "unit": "GB/s", "n_gpus": 1, "steps": iters, "warmup": 5,
        "ms_per_step": round(sum(r["hbm_us"] for r in q4) / 1e3, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "reference-published-shapes", "rows": rows_out,
                   "note": "rtx4090_published_GBps are the reference's cache-resident RTX 4090 figures; "
                           "host_GBps follows the reference's timing method on this GPU"},
        "roofline": {"bound": "hbm", "achieved": round(hbm, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(hbm / PEAK_HBM_GBS, 4), "traffic": None,
                     "kernel": "gemv_f32_kernel, Q4_K, the three published shapes, batch 1"},
        "cpu_baseline": None,
    }


def bench_gguf(E, synth, torch, args):
    """GGUF staging (the format step before the path): writes a Qwen3-8B-shaped
    GGUF (Q4_K token_embd and projections, Q5_K down, Q6_K output, f32 norms)
    with `--layers` layers to a temporary directory, then times opening it and
    staging every tensor into HBM through pinned double buffers, and the whole
    load into a decoder. The file is resident in the page cache (just written),
    so the figure is host-memory-to-HBM staging, not disk."""
    import tempfile

    import numpy as np

    from engine_amd import gguf_writer as W
    from engine_amd.gguf import GgufFile, load_qwen3_decode, qwen3_tensor_names, stage

    layers = args.layers
    md = [("general.architecture", W.STRING, "qwen3"), ("qwen3.block_count", W.U32, layers),
          ("qwen3.embedding_length", W.U32, HIDDEN), ("qwen3.feed_forward_length", W.U32, FFN),
          ("qwen3.attention.head_count", W.U32, 32), ("qwen3.attention.head_count_kv", W.U32, 8),
          ("qwen3.attention.key_length", W.U32, 128), ("qwen3.rope.freq_base", W.F32, 1.0e6),
          ("qwen3.attention.layer_norm_rms_epsilon", W.F32, 1.0e-6)]
    tensors = [("token_embd.weight", [HIDDEN, VOCAB], 12, synth.kquant_numpy(12, HIDDEN, VOCAB, seed=1)),
               ("output.weight", [HIDDEN, VOCAB], 14, synth.kquant_numpy(14, HIDDEN, VOCAB, seed=2)),
               ("output_norm.weight", [HIDDEN], 0, synth.gamma_numpy(HIDDEN, seed=3))]
    names = {"q": "attn_q", "k": "attn_k", "v": "attn_v", "o": "attn_output", "gate": "ffn_gate",
             "up": "ffn_up", "down": "ffn_down"}
    shared = {name: synth.kquant_numpy(t, k, n, seed=10 + i) for i, (name, t, k, n, _) in enumerate(LAYER)}
    for li in range(layers):
        for name, t, k, n, _ in LAYER:
            tensors.append((f"blk.{li}.{names[name]}.weight", [k, n], t, shared[name]))
        for nm, size in (("attn_norm", HIDDEN), ("ffn_norm", HIDDEN), ("attn_q_norm", 128), ("attn_k_norm", 128)):
            tensors.append((f"blk.{li}.{nm}.weight", [size], 0, synth.gamma_numpy(size, seed=li)))
    with tempfile.TemporaryDirectory() as tmp:
        path = os.path.join(tmp, "qwen3-8b-shaped.gguf")
        t0 = time.perf_counter()
        size = W.write(path, md, tensors)
        log(f"bench gguf: wrote {size / 1e9:.2f} GB in {time.perf_counter() - t0:.1f} s")
        del tensors, shared
        ctx = E.AmdContext(0)
        staged_bytes = 0
        runs = []
        for _ in range(3):
            t0 = time.perf_counter()
            g = GgufFile.open(path)
            t_open = time.perf_counter() - t0
            all_names = qwen3_tensor_names(layers) + ["output.weight"]
            staged = stage(ctx, g, all_names)
            dt = time.perf_counter() - t0
            staged_bytes = sum(g.tensor_data_range(n).stop - g.tensor_data_range(n).start for n in all_names)
            runs.append((dt, t_open))
            del staged
            g.close()
        dt, t_open = min(runs)
        gbs = staged_bytes / dt / 1e9
        log(f"bench gguf: open + stage {staged_bytes / 1e9:.2f} GB in {dt * 1e3:.1f} ms ({gbs:.1f} GB/s; "
            f"open {t_open * 1e3:.2f} ms)")
        t0 = time.perf_counter()
        dec, cfg, g, staged = load_qwen3_decode(ctx, path)
        t_load = time.perf_counter() - t0
        cache = E.AmdKvCache(ctx, cfg, 8)
        tok = dec.decode_step(cache, 7, 0)
        log(f"bench gguf: load_qwen3_decode {t_load * 1e3:.1f} ms; first token {tok}")
        dec.close()
    return {
        "metric": "GGUF open + staging into HBM, GB/s (page-cache resident file)",
        "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": 3, "warmup": 0,
        "ms_per_step": round(dt * 1e3, 3), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bytes", "data": "synthetic",
        "config": {"workload": "qwen3-8b-shaped-gguf-staging", "layers": layers, "file_bytes": size,
                   "staged_bytes": staged_bytes, "open_ms": round(t_open * 1e3, 3),
                   "load_decoder_ms": round(t_load * 1e3, 1)},
        "roofline": None, "cpu_baseline": None,
    }


def bench_prefill(E, synth, torch, args):
    """M = 512 bf16 tokens against Q4_K 4096->12288 and Q6_K 12288->4096
    (weights dequantised in registers, f16 MFMA, f32 accumulation)."""
    dev = torch.device("cuda:0")
    stream = torch.cuda.Stream()
    ctx = E.AmdContext(0, stream=stream)
    m = 512
    ctx.reserve_prefill(m, FFN, FFN)
    store = E.AmdWeightStore(ctx)
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    copies = 4
    shapes = (("q4k_4096x12288", 12, HIDDEN, FFN), ("q6k_12288x4096", 14, FFN, HIDDEN))
    out = {}
    total_flop, total_us = 0.0, 0.0
    for label, t, k, n in shapes:
        ws = []
        for c in range(copies):
            store.materialize_quantized(f"{label}{c}", [k, n], t, synth.kquant_torch(t, k, n, gen, dev))
            ws.append(store.quantized_tensor(f"{label}{c}"))
        kern = E.QwenGemvKernel.from_value_type(ctx, t)
        x = torch.randn(m, k, device=dev, generator=gen).to(torch.bfloat16)
        y = torch.empty(m * n, device=dev)

        def fn():
            for w in ws:
                kern.gemm_prefill(w, x, y, m)

        us = _graph_time_us(torch, stream, fn, max(2, args.steps // 10)) / copies
        flop = 2.0 * m * n * k
        out[label] = {"us": round(us, 2), "tflops": round(flop / us / 1e6, 1)}
        total_flop += flop
        total_us += us
        log(f"bench prefill: {label} M={m}: {us:.2f} us, {flop / us / 1e6:.1f} TFLOP/s")
    achieved = total_flop / total_us / 1e6
    return {
        "metric": "prefill matmul TFLOP/s (BASELINE config 3, M=512 bf16)",
        "value": round(achieved, 1), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(total_us / 1e3, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16-mfma-f32", "data": "synthetic",
        "config": {"workload": "prefill-m512", "shapes": out},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 1), "peak": PEAK_MFMA_F16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_MFMA_F16_TFLOPS, 4), "traffic": None,
                     "kernel": "act_f16_kernel + qgemm_tile_kernel (Q4_K 192-row tiles; Q6_K 256-row tiles, K split in 4, + qgemm_reduce_kernel), per call over both shapes"},
        "cpu_baseline": None,
    }


def bench_model(E, synth, torch, ctx, step, out_gamma, args):
    """BASELINE config 4 alone: the full Qwen3-8B-shaped decoder at batch 1 and 8."""
    res = model_decode_results(E, synth, torch, ctx, step, out_gamma, args)
    b1 = res[1]
    weight_bytes = step.bytes_per_step + HIDDEN // 256 * 144  # + one embedding row
    bytes_tok = weight_bytes + b1["kv_bytes_per_step"]
    achieved = bytes_tok * b1["tok_s"] / 1e9
    return {
        "metric": "Qwen3-8B-shaped Q4_K batch-1 decode tok/s (BASELINE config 4)",
        "value": b1["tok_s"], "unit": "tok/s", "n_gpus": 1, "steps": args.gen_tokens, "warmup": 1,
        "ms_per_step": b1["ms_per_step"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": ("f32" if args.gemv_mode == "warp" else "i8dot4-f32") + " GEMV, f16 KV, f32 attention",
        "data": "synthetic",
        "config": {"workload": "qwen3-8b-decode-model", "layers": args.layers, "context": args.context,
                   "generated": args.gen_tokens, "batches": res},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": None,
                     "kernel": "whole decode step (weights + KV cache per token)", "bytes_per_token": bytes_tok},
        "cpu_baseline": None,
    }


def _pct(values, q):
    """Nearest-rank percentile."""
    v = sorted(values)
    return v[max(0, min(len(v) - 1, int(-(-q * len(v) // 100)) - 1))] if v else None


def bench_serving(E, synth, torch, ctx, step, out_gamma, args):
    """The serving dispatcher under a burst (the reference's qwen_serving_bench
    burst mode): `concurrency` requests of `prompt_tokens` random prompt ids
    arrive together; a prefill-first scheduler submits at most
    `batch_tokens` prompt tokens per batch (prefill segments, the sampling row
    on each prompt's last segment), then whole decode batches; every batch is
    one submission polled to completion through AmdBackend. TTFT counts from
    the burst's arrival; ITL between a request's successive tokens."""
    import numpy as np
    from engine_amd import serving as S

    members = max(8, args.prefill_chunk)
    dec, cfg = build_decoder(E, synth, torch, ctx, step, out_gamma, args.layers, args.seed, members)
    cap = args.prompt_tokens + args.tokens
    per_seq = S.qwen3_kv_bytes(cfg, cap)
    disp = S.AmdServingDispatcher(dec, args.concurrency, kv_budget_bytes=per_seq * args.concurrency)
    if args.prefill_chunk:
        disp.with_prefill_chunk(args.prefill_chunk)
    if args.prompt_prefill:
        disp.with_prompt_prefill(args.prompt_prefill)
    caps = S.BackendCapabilities("rocm", 0, "rocm", torch.cuda.get_device_properties(0).total_memory)
    plan = S.ExecutionPlan("qwen3-8b-shaped", "rocm", 0, 1, frozenset((S.Phase.PREFILL, S.Phase.DECODE)))
    backend = S.AmdBackend(caps, disp)
    rng = np.random.default_rng(args.seed + 7)

    def run_burst(tokens):
        reqs = [{"id": 10_000 * (run_burst.n + 1) + i, "prompt": [int(t) for t in rng.integers(0, VOCAB, args.prompt_tokens)],
                 "done": 0, "out": [], "times": []} for i in range(args.concurrency)]
        run_burst.n += 1
        for r in reqs:
            r["state"] = S.InferenceStateSet(r["id"], kv_tokens=cap)
        t0 = time.perf_counter()
        batches = 0
        while any(len(r["out"]) < tokens for r in reqs):
            segs, states, owners, budget = [], [], [], args.batch_tokens
            for r in reqs:
                left = len(r["prompt"]) - r["done"]
                if left > 0 and budget > 0:
                    n = min(left, budget)
                    last = n == left
                    segs.append(S.ExecutionSegment(r["id"], S.Phase.PREFILL, n, r["done"],
                                                   tuple(r["prompt"][r["done"]:r["done"] + n]),
                                                   S.SamplingParams.greedy() if last else None))
                    budget -= n
                    states.append(r["state"])
                    owners.append(r)
            if not segs:
                for r in reqs:
                    if len(r["out"]) < tokens:
                        pos = len(r["prompt"]) + len(r["out"]) - 1
                        segs.append(S.ExecutionSegment(r["id"], S.Phase.DECODE, 1, pos, (r["out"][-1],),
                                                       S.SamplingParams.greedy()))
                        states.append(r["state"])
                        owners.append(r)
            batch = S.ExecutionBatch(tuple(segs))
            ev = backend.wait(backend.submit(plan, batch, states))
            now = time.perf_counter() - t0
            S.commit_batch(batch, states)
            batches += 1
            for r, seg, e in zip(owners, segs, ev.events):
                if seg.phase == S.Phase.PREFILL:
                    r["done"] += seg.token_count
                if e.output_token is not None:
                    r["out"].append(e.output_token)
                    r["times"].append(now)
        wall = time.perf_counter() - t0
        for r in reqs:
            backend.release_inference_state(r["state"])
        return reqs, wall, batches

    run_burst.n = 0
    log(f"bench serving: warm-up burst ({args.concurrency} x {args.prompt_tokens} prompt tokens, 2 tokens)")
    run_burst(2)
    log(f"bench serving: timed burst ({args.concurrency} x {args.prompt_tokens} prompt, {args.tokens} tokens, "
        f"prefill chunk {args.prefill_chunk or 'off'}, prompt prefill {args.prompt_prefill or 'off'})")
    reqs, wall, batches = run_burst(args.tokens)
    ttft = [r["times"][0] for r in reqs]
    itl = [b - a for r in reqs for a, b in zip(r["times"], r["times"][1:])]
    first_all = max(ttft)
    decode_tokens = sum(len(r["out"]) - 1 for r in reqs)
    decode_s = wall - first_all
    out_tokens = sum(len(r["out"]) for r in reqs)
    prompt_total = args.concurrency * args.prompt_tokens
    used, reusable = disp.state_bytes()
    # what 288 GB holds: sequences of the full 4096-token context beside the weights
    full = E.AmdQwen3Config(layers=36)
    per4k = S.qwen3_kv_bytes(full, 4096)
    mem = S.plan_memory(ctx, per4k, 1)
    fit = (mem.free_before_preparation_bytes - (512 << 20)) // per4k
    result = {
        "metric": "Qwen3-8B-shaped serving output tok/s (burst through the serving dispatcher)",
        "value": round(out_tokens / wall, 1), "unit": "tok/s", "n_gpus": 1, "steps": batches, "warmup": 1,
        "ms_per_step": round(wall * 1e3 / batches, 3), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "data": "synthetic",
        "dtype": ("f32" if args.gemv_mode == "warp" else "i8dot4-f32") + " GEMV, f16 KV, f32 attention",
        "config": {"workload": "qwen3-8b-serving-burst", "layers": args.layers, "concurrency": args.concurrency,
                   "prompt_tokens": args.prompt_tokens, "output_tokens": args.tokens,
                   "prefill_chunk": args.prefill_chunk, "prompt_prefill": args.prompt_prefill,
                   "batch_tokens": args.batch_tokens,
                   "grouped_decode": False},
        "serving": {"wall_s": round(wall, 3), "batches": batches,
                    "prefill_tok_s": round(prompt_total / first_all, 1),
                    "decode_tok_s": round(decode_tokens / decode_s, 1) if decode_s > 0 else None,
                    "ttft_ms": {"mean": round(1e3 * sum(ttft) / len(ttft), 1), "p50": round(1e3 * _pct(ttft, 50), 1),
                                "max": round(1e3 * max(ttft), 1)},
                    "itl_ms": {"mean": round(1e3 * sum(itl) / len(itl), 3) if itl else None,
                               "p50": round(1e3 * _pct(itl, 50), 3) if itl else None,
                               "p99": round(1e3 * _pct(itl, 99), 3) if itl else None,
                               "max": round(1e3 * max(itl), 3) if itl else None},
                    "kv_bytes_per_sequence": per_seq, "kv_state_bytes_after_release": [used, reusable]},
        "memory_288gb": {"free_bytes_now": mem.free_before_preparation_bytes,
                         "qwen3_8b_kv_bytes_per_token": S.qwen3_kv_bytes(full, 1),
                         "kv_bytes_per_4096_token_sequence": per4k,
                         "additional_4096_token_sequences_that_fit": int(fit)},
        "roofline": None, "cpu_baseline": None,
    }
    disp.close()
    dec.close()
    return result


def bench_mfma_peak(E, synth, torch, args):
    """The measured dense peak of the matrix-core instructions (the published
    2.5 PFLOP/s f16 / bf16 figure checked with a microbenchmark):
    ribn_amd_probe_mfma_peak, a full grid of four waves per SIMD issuing
    independent MFMAs on register operands, median of 5 runs."""
    import ctypes
    ctx = E.AmdContext(0)
    kinds = {0: "v_mfma_f32_16x16x32_f16", 1: "v_mfma_f32_32x32x16_f16", 2: "v_mfma_f32_16x16x32_bf16",
             3: "v_mfma_f32_16x16x4_f32"}
    published = {0: 2500.0, 1: 2500.0, 2: 2500.0, 3: 157.3}
    res = {}
    for kind, name in kinds.items():
        runs = []
        for _ in range(5):
            out = ctypes.c_double()
            st = ctx._lib.ribn_amd_probe_mfma_peak(ctx.handle, kind, 20000, ctypes.byref(out))
            if st != 0:
                raise RuntimeError(f"MFMA probe failed with status {st}")
            runs.append(out.value)
        runs.sort()
        res[name] = {"tflops": round(runs[2], 1), "published_tflops": published[kind],
                     "of_published": round(runs[2] / published[kind], 4)}
        log(f"bench mfma-peak: {name}: {runs[2]:.1f} TFLOP/s ({runs[2] / published[kind]:.1%} of {published[kind]})")
    f16 = res["v_mfma_f32_16x16x32_f16"]["tflops"]
    return {"metric": "MI355X dense f16 MFMA peak, measured (v_mfma_f32_16x16x32_f16)", "value": f16,
            "unit": "TFLOP/s", "n_gpus": 1, "steps": 5, "warmup": 1, "ms_per_step": None, "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "f16", "data": "synthetic",
            "config": {"workload": "mfma-peak", "iterations": 20000, "waves_per_simd": 4, "kinds": res},
            "roofline": {"bound": "mfma", "achieved": f16, "peak": PEAK_MFMA_F16_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(f16 / PEAK_MFMA_F16_TFLOPS, 4), "traffic": None},
            "cpu_baseline": None}


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "gemv_f32_q4k_gate_up_traffic.md")


def measured_traffic():
    """HBM bytes per gate+up launch from the committed rocprofv3 FETCH_SIZE and
    WRITE_SIZE passes, when they were taken on the current kernel sources."""
    try:
        from engine_amd.profiling import source_hash
        fields = {}
        with open(TRAFFIC_PROFILE) as f:
            for line in f:
                if "=" in line and line.strip().startswith(("traffic_bytes_per_launch", "source_hash")):
                    k, v = line.split("=", 1)
                    fields[k.strip()] = v.strip().strip("`")
        if fields.get("source_hash") != source_hash():
            return None
        return int(fields["traffic_bytes_per_launch"])
    except (OSError, KeyError, ValueError):
        return None


def _cpu_model():
    """The host CPU as `lscpu` reports it: model name, vendor family / model /
    stepping (identifying the part where a VM shortens the name, e.g. family 26
    is AMD Zen 5, 25 Zen 3/4), sockets, cores, threads and L3. Falls back to
    /proc/cpuinfo for the name."""
    keys = {"Model name": "name", "Vendor ID": "vendor", "CPU family": "family", "Model": "model",
            "Stepping": "stepping", "Socket(s)": "sockets", "Core(s) per socket": "cores_per_socket",
            "Thread(s) per core": "threads_per_core", "L3": "l3", "L3 cache": "l3", "CPU max MHz": "max_mhz",
            "Hypervisor vendor": "hypervisor"}
    info = {}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            k, _, v = line.partition(":")
            k = k.strip()
            if k in keys and keys[k] not in info and v.strip():
                info[keys[k]] = v.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    if "name" not in info:
        try:
            with open("/proc/cpuinfo") as f:
                for line in f:
                    if line.startswith("model name"):
                        info["name"] = line.split(":", 1)[1].strip()
                        break
        except OSError:
            pass
    info.setdefault("name", "unknown")
    info["cpus_usable"] = len(os.sched_getaffinity(0))
    return info


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layers", type=int, default=36)
    ap.add_argument("--seed", type=int, default=2024)
    ap.add_argument("--no-graph", action="store_true", help="issue launches eagerly instead of replaying a HIP graph")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--gemv-mode", choices=tuple(GEMV_MODES), default="warp",
                    help="GEMV arithmetic: warp (f32 activations, default) or fixed16 (opt-in block fixed point)")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--workload", choices=("decode", "batched", "prefill", "model", "q8_1", "gguf", "serving",
                                           "mfma-peak", "published"),
                    default="decode",
                    help="decode: BASELINE config 1 (the headline line, default, which also carries the "
                         "config-4 tok/s); batched: config 2 (FFN at M = 1, 4, 16, 64); prefill: config 3 "
                         "(M = 512 bf16 matmuls); model: config 4 alone (full decoder, batch 1 and 8); q8_1: "
                         "the Q8_1 integer-dot projections (pack + GEMV) at batch 1 and 8; gguf: GGUF "
                         "open + staging of a Qwen3-8B-shaped file (--layers layers); mfma-peak: the "
                         "measured dense peak of the matrix-core instructions the prefill uses; published: the "
                         "reference's own GEMV bench shapes (int_dot_bench), batch 1 and 8, beside its RTX 4090 "
                         "figures")
    ap.add_argument("--context", type=int, default=2048, help="config 4: prompt tokens before generation")
    ap.add_argument("--gen-tokens", type=int, default=128, help="config 4: greedy tokens timed")
    ap.add_argument("--prompt-chunk", type=int, default=2048,
                    help="config 4: prompt tokens per prefill-matmul chunk (0: serial single-token prefill)")
    ap.add_argument("--no-model", action="store_true", help="skip the config-4 full-decoder measurement")
    ap.add_argument("--no-batched", action="store_true", help="skip the config-2 M = 16 / 64 FFN figures")
    ap.add_argument("--concurrency", type=int, default=8, help="serving: requests in the burst")
    ap.add_argument("--prompt-tokens", type=int, default=257, help="serving: prompt tokens per request")
    ap.add_argument("--tokens", type=int, default=32, help="serving: output tokens per request")
    ap.add_argument("--prefill-chunk", type=int, default=8, help="serving: prefill chunk members (0: serial)")
    ap.add_argument("--batch-tokens", type=int, default=128, help="serving: prompt tokens per scheduler batch")
    ap.add_argument("--prompt-prefill", type=int, default=2048,
                    help="serving: prefill prefixes of 16+ tokens on the prefill matmul in chunks of this many "
                         "tokens (0: off, the prefill-chunk / serial path)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="after the timed work, copy a MIB-MiB device buffer three times: a kernel of known "
                         "traffic that scales rocprofv3 FETCH_SIZE / WRITE_SIZE onto bytes")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build measures one GPU: the k-quant decode path runs on a single "
                                   "MI355X; multi-GPU sharding is a design note only", "n_gpus": args.gpus}))
        sys.exit(2)

    import torch

    import engine_amd as E
    from engine_amd import synth

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    torch.cuda.set_device(0)
    if args.workload in ("batched", "prefill", "q8_1", "gguf", "mfma-peak", "published"):
        result = {"batched": bench_batched, "prefill": bench_prefill, "q8_1": bench_q8_1,
                  "gguf": bench_gguf, "mfma-peak": bench_mfma_peak, "published": bench_published}[args.workload](
            E, synth, torch, args)
        print(json.dumps(result), flush=True)
        return
    log(f"bench: generating {args.layers} layers + lm_head of synthetic weights on the device")
    weights, head, out_gamma, acts = build_model(E, synth, torch, args.layers, args.seed)
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    ctx = E.AmdContext(0, stream=stream)
    step = DecodeGemvStep(E, torch, ctx, weights, head, out_gamma, acts, GEMV_MODES[args.gemv_mode])
    build_decoder.mode = args.gemv_mode
    log(f"bench: {step.bytes_per_step / 1e9:.3f} GB of algorithmic traffic per step")

    if args.workload == "model":
        print(json.dumps(bench_model(E, synth, torch, ctx, step, out_gamma, args)), flush=True)
        return
    if args.workload == "serving":
        print(json.dumps(bench_serving(E, synth, torch, ctx, step, out_gamma, args)), flush=True)
        return

    gu_bytes = 2 * (launch_bytes(12, HIDDEN, FFN) - 4 * HIDDEN) + 4 * HIDDEN

    def measure(mode):
        """ms per step of the 36-layer + lm_head GEMV chain, and mean us per
        gate+up group launch (timed live with HIP events over back-to-back
        launches on the stream they run on), in one GEMV mode."""
        step.set_mode(GEMV_MODES[mode])
        with torch.cuda.stream(stream):
            step.run()  # eager warm-up (and validation of every launch)
        torch.cuda.synchronize()
        graph = None if args.no_graph else capture(torch, stream, step.run)
        graph_gu = None if args.no_graph else capture(torch, stream, step.run_gate_up)
        one = graph.replay if graph is not None else step.run
        with torch.cuda.stream(stream):
            for _ in range(args.warmup):
                one()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            start.record(stream)
            for _ in range(args.steps):
                one()
            end.record(stream)
        torch.cuda.synchronize()
        ms = start.elapsed_time(end) / args.steps
        reps = 5
        gate_up = graph_gu.replay if graph_gu is not None else step.run_gate_up
        with torch.cuda.stream(stream):
            gate_up()
            ev = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
            ev[0].record(stream)
            for r in range(reps):
                gate_up()
                ev[r + 1].record(stream)
        torch.cuda.synchronize()
        # mean us per gate+up launch over each replay of the 36 launches
        per = sorted(ev[r].elapsed_time(ev[r + 1]) * 1e3 / args.layers for r in range(reps))
        mean = ev[0].elapsed_time(ev[reps]) * 1e3 / (reps * args.layers)
        return ms, mean, graph is not None, per[reps // 2], per[0]

    # The opt-in fixed-point mode first (for comparison), then the headline mode.
    other = "fixed16" if args.gemv_mode == "warp" else "warp"
    ms_o, us_o, _, _, _ = measure(other)
    log(f"bench: {other} GEMV mode (comparison): {ms_o:.4f} ms/step, "
        f"{step.bytes_per_step / (ms_o * 1e-3) / 1e9:.1f} GB/s, gate+up {us_o:.3f} us")
    ms_step, us_launch, graphed, us_median, us_min = measure(args.gemv_mode)
    gbs = step.bytes_per_step / (ms_step * 1e-3) / 1e9
    log(f"bench: {args.gemv_mode} GEMV mode: {ms_step:.4f} ms/step, {gbs:.1f} GB/s, gate+up {us_launch:.3f} us")
    achieved = gu_bytes / (us_launch * 1e-6) / 1e9
    roofline = {
        "bound": "hbm",
        "kernel": ("gemv_f32_kernel<Q4_K, 1 member, fused RMSNorm>" if args.gemv_mode == "warp" else
                   "gemv_wave_kernel<Q4_K, 1 member, fused RMSNorm>") + ": gate+up group, 4096->2x12288",
        "achieved": round(achieved, 1),
        "peak": PEAK_HBM_GBS,
        "unit": "GB/s",
        "frac": round(achieved / PEAK_HBM_GBS, 4),
        "traffic": measured_traffic(),
        "avg_launch_us": round(us_launch, 3),
        "median_launch_us": round(us_median, 3),  # of the 5 replays' means
        "min_launch_us": round(us_min, 3),
        "bytes_per_launch": gu_bytes,
    }

    if args.calibrate_copy > 0:
        src = torch.empty(args.calibrate_copy << 20, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()

    model = None
    if not args.no_model:
        model = model_decode_results(E, synth, torch, ctx, step, out_gamma, args)

    batched = None
    if not args.no_batched:
        # BASELINE config 2 at the sizes the f32-faithful matrix-core GEMV serves (its own line:
        # --workload batched)
        per_m, _, _ = batched_ffn_times(E, synth, torch, args, ms=(16, 64), compare=False)
        batched = {"us_per_ffn": {str(m): per_m[m]["warp"]["us_per_ffn"] for m in per_m},
                   "tokens_per_s": {str(m): per_m[m]["warp"]["tokens_per_s"] for m in per_m},
                   "dtype": "f32 (f16 MFMA on exact two-piece activations, f32 accumulation)",
                   "workload": "qwen3-8b-ffn-batched (gate/up Q4_K grouped + down Q5_K, 8 layers cycled)"}

    cpu = None
    if not args.no_cpu_baseline:
        log("bench: timing the CPU baseline")
        cpu = cpu_baseline(args.cpu_seconds)

    result = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        # warp: f32 activations x weights dequantised to f32 in registers, f32 FMAs;
        # fixed16: 4..6-bit quants x 16-bit fixed-point activations (v_dot4, int32), scales f32
        "dtype": "f32" if args.gemv_mode == "warp" else "i8dot4-f32",
        "data": "synthetic",
        "hbm_frac": round(gbs / PEAK_HBM_GBS, 4),
        # the full decoder (embedding, 36 layers with attention
        # over a 2048-token f16 KV cache, lm_head, argmax), greedy, graph-replayed
        "decode_tok_s": model[1]["tok_s"] if model else None,
        "decode_tok_s_b8": model[8]["tok_s"] if model else None,
        "decode_model": model,
        "batched_ffn": batched,
        "gemv_chain_tok_s": round(1000.0 / ms_step, 2),
        "gemv_mode": args.gemv_mode,
        "comparison_mode": {"gemv_mode": other, "dtype": "i8dot4-f32" if other == "fixed16" else "f32",
                            "value": round(step.bytes_per_step / (ms_o * 1e-3) / 1e9, 2), "unit": "GB/s",
                            "ms_per_step": round(ms_o, 5), "gate_up_us": round(us_o, 3)},
        "config": {
            "workload": "qwen3-8b-decode-gemv-b1",
            "layers": args.layers,
            "hidden": HIDDEN,
            "ffn": FFN,
            "projections": "q,k,v,o,gate,up Q4_K; down Q5_K; lm_head Q6_K 151936x4096",
            "rmsnorm": "fused into the q/k/v group, gate/up group and lm_head activation load, eps 1e-6",
            "bytes_per_step": step.bytes_per_step,
            "launches_per_step": 4 * args.layers + 1,
            "hip_graph": graphed,
            "batch": 1,
        },
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
