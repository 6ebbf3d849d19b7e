#!/usr/bin/env python3
"""Benchmark of the MTP speculative-decoding verify step on one MI355X.

One step = the reference's Scheduler._verify_step with MTP drafts (qwen38_inf2/scheduler.py:160-193, 269-301) for
all 64 rows: 3 MTP calls and 3 one-group head passes to draft 3 tokens per row, the 64-layer verify of 4 tokens per
row (512-token contexts), the head's group maxima and exact top-4-group recheck over 256 rows, greedy acceptance and
the state advance. It runs as one library call, `q38_spec_step_graph` (the step captured once per gated-delta parity
as a HIP graph and replayed), on torch's current HIP stream; `ms_per_step_launches` is the same step as individual
launches (`q38_spec_step`). Inputs and state are resident in HBM. Weights are seeded random-init FP8 e4m3 (+E8M0 per 32) of the Qwen3.8-27B shapes; there is no
checkpoint.

    python bench.py [--steps K] [--warmup W] [--no-cpu-baseline] [--decode | --prefill | --config 3|4] [--mxfp4] [--kv-fp8]

prints one JSON line. `value` is accepted tokens per second (the sum of every row's accepted count, which advances
its position, over the timed steps). `roofline` is the dominant kernel, the MLP gate/up projection (gemm_kernel with
the SwiGLU epilogue, 2 x 17408 x 5120 FP8 weights against 256 tokens): HIP events around each of its launches inside
`--steps` further speculative steps, on the stream it runs on (q38_kernel_timer); `traffic` is its HBM bytes per
launch from the committed counter summary in profiles/.
`step_roofline` is the whole step's algorithmic HBM bytes over its time. `cpu_baseline` is the CPU oracle (this
repository's restatement of the reference's CPU path) on a bounded sample: one 27B block (3 gated-delta + 1 attention
layer) of the verify at the same B, K and context, scaled x16 to 64 layers, without the MTP and head passes.

`--decode` measures the one-token decode graph instead (`q38_decode`: the reference's step graph in its decode form,
model.py:983-995 with GatedDeltaNetStep.forward and FullAttentionStep.forward) over the same 64 rows from 512-token
contexts, one token per row per step: `value` is tokens per second, `roofline` the step's algorithmic HBM bytes
(weights, scales, gated-delta and conv state read + written, KV read over the context, inputs and outputs) over its
time, and `cpu_baseline` the CPU oracle's decode of one block, x16.

`--prefill` measures the prefill form (`q38_prefill`, model.py:476-521 and 704-783): one row's prompt of 4096 tokens in
two chunks of 2048 (the second one attending to the first's 2048 cached positions) plus the MTP layer's cache-only
prefill of each chunk: `value` is prompt tokens per second, `roofline` the projections' bf16 MFMA work (2 x tokens x
every projection weight; attention's own products left out) over the time against the dense bf16 peak, and `cpu_baseline` the CPU oracle's prefill of one block
on a 512-token chunk, x16.

`--config 3` / `--config 4` measure BASELINE configs 3 and 4 at block level (one 27B block of 3 gated-delta + 1
attention layer, `q38_verify`): B=16, K=4 from 32768 cached positions (HBM-bound: `roofline` in GB/s), or B=256, K=8
from 4096 (near the MFMA balance: `roofline` in TFLOP/s of the block's matrix work); `value` is verify tokens per
second through the block, `cpu_baseline` the CPU oracle's verify of the same block.

`--mxfp4` binds the 64 decoder layers' projections as MXFP4 (the checkpoint's E2M1 nibbles + E8M0 scales, read by the
GEMMs directly: half the weight bytes of e4m3), the seeded e4m3 weights requantized; the MTP layer and the head stay
e4m3, as an MXFP4 checkpoint holds them in bf16. The algorithmic bytes count the decoder weights at 4.25 bits.

`--context N` starts every row from N cached positions instead of 512 (for long-context runs of the verify and
decode steps; run those with --no-cpu-baseline). `--kv-fp8` keeps every attention layer's KV cache (the MTP layer's too) as e4m3 bytes with per-layer bf16 scales (the
reference's kv_cache_format "fp8"): half the KV bytes; the synthetic caches are encoded with seeded scales.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "qwen38-27b-aws_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

HBM_PEAK_GBS = 8000.0     # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
FP8_PEAK_TFLOPS = 5000.0  # MI355X dense FP8 MFMA


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def fp8_bytes(n: int, k: int) -> int:
    return n * k + n * k // 32


def fp4_bytes(n: int, k: int) -> int:
    return n * k // 2 + n * k // 32


def algorithmic_bytes(cfg, batch: int, tokens: int, context: int, mxfp4: bool = False, kv8: bool = False) -> dict:
    """Compulsory HBM bytes of one step, each counted once: FP8 weights + E8M0 scales of every projection streamed,
    bf16 small weights, gated-delta state and conv state read + written, KV read over each row's context plus the
    step's own K/V written, the head read once per pass plus the recheck rows, the MTP layer per call, inputs/outputs."""
    h, inter, v = cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size
    hv, hk, d, c = cfg.linear_num_value_heads, cfg.linear_num_key_heads, cfg.linear_key_head_dim, cfg.linear_conv_dim
    hq, hkv, hd = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    t = batch * tokens
    wb = fp4_bytes if mxfp4 else fp8_bytes  # the decoder layers' projections
    mlp = wb(2 * inter, h) + wb(h, inter)
    gdn_w = wb(c + hv * d, h) + wb(h, hv * d) + mlp + 2 * hv * h * 2 + c * 4 * 2
    attn_w = wb(hq * hd * 2 + 2 * hkv * hd, h) + wb(h, hq * hd) + mlp
    attn_w8 = fp8_bytes(hq * hd * 2 + 2 * hkv * hd, h) + fp8_bytes(h, hq * hd) + fp8_bytes(2 * inter, h) + fp8_bytes(h, inter)
    n_gdn = sum(1 for k in cfg.layer_types if k == "linear_attention")
    n_attn = cfg.num_hidden_layers - n_gdn
    weights = n_gdn * gdn_w + n_attn * attn_w
    state = n_gdn * batch * (hv * d * d * 2 * 2 + c * 3 * 2 * 2)
    kv_elem = 1 if kv8 else 2  # bytes per cached element
    kv_read = batch * hkv * context * hd * 2 * kv_elem
    kv = n_attn * (kv_read + t * hkv * hd * 2 * kv_elem)
    io = t * h * 2 * 2
    head_pass = fp8_bytes(v, h)
    head = 4 * head_pass + (t * 4 + 3 * batch) * 32 * (h + h // 32)
    mtp_w = fp8_bytes(h, 2 * h) + attn_w8
    mtp = 3 * (mtp_w + kv_read + t * hkv * hd * 2 * kv_elem + 3 * t * h * 2)
    total = weights + state + kv + io + head + mtp
    return {"total": total, "weights": weights, "state": state, "kv": kv, "head": head, "mtp": mtp, "io": io}


def decode_bytes(cfg, batch: int, context: int, mxfp4: bool = False, kv8: bool = False) -> int:
    """Compulsory HBM bytes of one decode step (no head, no MTP): as `algorithmic_bytes` with one token per row."""
    b = algorithmic_bytes(cfg, batch, 1, context, mxfp4, kv8)
    return b["weights"] + b["state"] + b["kv"] + b["io"]


def build(cfg, batch: int, tokens: int, max_seq_len: int, context: int, seed: int, mxfp4: bool = False, kv8: bool = False,
          mfma: str = "bf16"):
    import torch

    from qwen38_amd import synth
    from qwen38_amd.quant import encode_kv
    from qwen38_amd.steps import Engine

    dev = "cuda"
    engine = Engine(cfg, batch, tokens, max_seq_len, mtp=True, device=dev, weight_format="mxfp4" if mxfp4 else "e4m3",
                    kv_cache_format="fp8" if kv8 else "bf16", projection_mfma=mfma)

    def set_kv(layer, name):
        kv = synth.kv_states(cfg, batch, max_seq_len, ctx, seed, name, dev)
        if kv8:
            ks, vs = synth.kv_scales(cfg, seed, name, dev)
            engine.set_kv_scales(layer, ks, vs)
            kv = {"k_cache": encode_kv(kv["k_cache"], ks), "v_cache": encode_kv(kv["v_cache"], vs)}
        engine.set_kv(layer, kv["k_cache"], kv["v_cache"])

    started = time.time()
    specs = synth.model_specs(cfg, mtp=True, head=True)

    def weights():
        for n, spec in enumerate(specs):
            if n % 100 == 0:
                log(f"weights {n}/{len(specs)} ({time.time() - started:.0f}s)")
            yield spec.name, synth.make(spec, seed, dev)

    engine.load(synth.to_mxfp4(weights()) if mxfp4 else weights())
    ctx = [context] * batch
    for i, kind in enumerate(cfg.layer_types):
        if kind == "linear_attention":
            engine.set_gdn(i, synth.gdn_states(cfg, batch, tokens, seed, f"state.{i}", dev))
        else:
            set_kv(i, f"kv.{i}")
    set_kv(engine.mtp_layer, "kv.mtp")
    torch.cuda.synchronize()
    log(f"model and state ready in {time.time() - started:.0f}s")
    g = torch.Generator(device=dev).manual_seed(seed)
    state = {
        "position": torch.full((batch,), context, dtype=torch.int32, device=dev),
        "index": torch.full((batch,), context - 1, dtype=torch.int32, device=dev),
        "match": torch.zeros(batch, dtype=torch.int32, device=dev),
        "accepted": torch.ones(batch, dtype=torch.int32, device=dev),
        "active": torch.ones(batch, dtype=torch.float32, device=dev),
        "hidden": synth.hidden_states((batch, tokens, cfg.hidden_size), seed, "bench.hidden", dev),
        "picks": torch.randint(0, cfg.vocab_size, (batch, tokens), generator=g, device=dev, dtype=torch.int32),
        "drafts": torch.zeros(batch, tokens - 1, dtype=torch.int32, device=dev),
    }
    return engine, state


TRAFFIC_SUMMARY = ROOT / "profiles" / "gemm_swiglu_256x34816x5120_traffic.md"


def profiled_traffic() -> int | None:
    """HBM bytes per launch of the roofline kernel from its committed counter summary: FETCH_SIZE and WRITE_SIZE of the
    same kernel on this workload (rocprofv3 --pmc, one counter per run), each scaled by what the counter reads for a
    copy of known size in the same run. None when the summary is absent."""
    try:
        for line in TRAFFIC_SUMMARY.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":", 1)[1])
    except (OSError, ValueError):
        pass
    return None


def cpu_baseline(cfg_block, batch: int, tokens: int, max_seq_len: int, context: int, seed: int, accepted_per_step: float,
                 n_blocks: int) -> dict:
    """The CPU oracle on one block of the same verify (bf16, all host threads), timed once after one warm-up."""
    import torch

    from oracle import model as om
    from qwen38_amd import synth
    from qwen38_amd.generate import verify_inputs

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    values = {}
    for spec in synth.model_specs(cfg_block, mtp=False, head=False):
        v = synth.make(spec, seed, "cuda")
        values[spec.name] = tuple(x.cpu() for x in v) if isinstance(v, tuple) else v.cpu()
    layers = []
    for i in range(cfg_block.num_hidden_layers):
        prefix = f"layers.{i}."
        layers.append({n[len(prefix):]: (om.FP8Weight(*v) if isinstance(v, tuple) else v) for n, v in values.items() if n.startswith(prefix)})
    states = []
    for i, kind in enumerate(cfg_block.layer_types):
        if kind == "linear_attention":
            states.append({k: v.cpu() for k, v in synth.gdn_states(cfg_block, batch, tokens, seed, f"cpu.{i}", "cuda").items()})
        else:
            states.append({k: v.cpu() for k, v in synth.kv_states(cfg_block, batch, max_seq_len, [context] * batch, seed, f"cpu.{i}", "cuda").items()})
    x = synth.hidden_states((batch, tokens, cfg_block.hidden_size), seed, "cpu.x")
    inp = verify_inputs(cfg_block, [context] * batch, tokens, max_seq_len, torch.bfloat16, [True] * batch, [1] * batch)
    times = []
    for _ in range(2):
        started = time.perf_counter()
        om.step_verify(cfg_block, layers, states, x, inp["cos"], inp["sin"], inp["position"], inp["active"], inp["accepted"])
        times.append(time.perf_counter() - started)
        log(f"cpu block {times[-1]:.2f}s")
    del layers, states, values

    # The MTP layer: one call over the B x K rows, three per step (the device step calls it with every row's K slots).
    mtp_vals = {}
    for spec in synth.mtp_specs(cfg_block) + [s for s in synth.head_specs(cfg_block) if s.name == "head.norm_weight"]:
        v = synth.make(spec, seed, "cuda")
        mtp_vals[spec.name] = tuple(t.cpu() for t in v) if isinstance(v, tuple) else v.cpu()
    mw = {n[len("mtp."):]: (om.FP8Weight(*v) if isinstance(v, tuple) else v) for n, v in mtp_vals.items() if n.startswith("mtp.")}
    mw["final_norm_weight"] = mtp_vals["head.norm_weight"]
    mst = {k: v.cpu() for k, v in synth.kv_states(cfg_block, batch, max_seq_len, [context] * batch, seed, "cpu.mtp", "cuda").items()}
    minp = verify_inputs(cfg_block, [context] * batch, tokens, max_seq_len, torch.bfloat16, [True] * batch, [0] * batch)
    emb = synth.hidden_states((batch, tokens, cfg_block.hidden_size), seed, "cpu.e")
    mtp_s = 0.0
    for _ in range(2):
        started = time.perf_counter()
        om.mtp_forward(cfg_block, mw, mst, x, emb, minp["cos"], minp["sin"], minp["position"], minp["active"])
        mtp_s = time.perf_counter() - started
    log(f"cpu MTP call {mtp_s:.2f}s")
    del mw, mst, mtp_vals

    # The head's group maxima: HEAD_ROWS rows against a 1/HEAD_VOCAB_PART slice of lm_head, scaled to the step's
    # B x K verify rows plus three draft passes of B rows (linear in rows and in vocabulary).
    head_rows, part = 16, 8
    vs = cfg_block.vocab_size // part // 32 * 32
    spec = [s for s in synth.head_specs(cfg_block) if s.name == "head.lm_head"][0]
    spec = synth.Spec(spec.name, spec.kind, (vs, cfg_block.hidden_size))
    coded, scales = (t.cpu() for t in synth.make(spec, seed, "cuda"))
    lm = om.FP8Weight(coded, scales)
    hx = synth.hidden_states((head_rows, 1, cfg_block.hidden_size), seed, "cpu.h")
    nw = synth.make([s for s in synth.head_specs(cfg_block) if s.name == "head.norm_weight"][0], seed, "cpu")
    lm.dense_t()
    started = time.perf_counter()
    om.head_group_maxima(cfg_block, nw, lm, hx)
    head_sample = time.perf_counter() - started
    head_rows_step = batch * tokens + (tokens - 1) * batch
    head_s = head_sample * part * head_rows_step / head_rows
    log(f"cpu head sample {head_sample:.2f}s ({head_rows} rows, 1/{part} of the vocabulary) -> {head_s:.2f}s per step")
    step = times[-1] * n_blocks + 3 * mtp_s + head_s
    cpu_name = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_name = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": accepted_per_step / step,
        "unit": "accepted tokens/s",
        "cores": threads,
        "kind": "port",
        "sample": f"the CPU oracle in bf16, timed after one warm-up: one block (3 gated-delta + 1 attention layer) of the "
        f"B={batch}, K={tokens}, context-{context} verify ({times[-1]:.2f} s) x{n_blocks} for 64 layers, plus 3 MTP calls "
        f"over the B x K rows ({mtp_s:.2f} s each), plus the head's group maxima for {head_rows_step} rows scaled from "
        f"{head_rows} rows against 1/{part} of lm_head ({head_sample:.2f} s -> {head_s:.2f} s): {step:.2f} s per step; "
        f"host {cpu_name}",
    }


def cpu_decode_baseline(cfg_block, batch: int, max_seq_len: int, context: int, seed: int, n_blocks: int) -> dict:
    """The CPU oracle's decode step on one block (bf16, all host threads), timed once after one warm-up."""
    import torch

    from oracle import model as om
    from qwen38_amd import synth
    from qwen38_amd.generate import batch_step_inputs

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    layers = []
    for i in range(cfg_block.num_hidden_layers):
        prefix = f"layers.{i}."
        w = {}
        for spec in synth.layer_specs(cfg_block, i):
            v = synth.make(spec, seed, "cuda")
            w[spec.name[len(prefix):]] = om.FP8Weight(*(x.cpu() for x in v)) if isinstance(v, tuple) else v.cpu()
        layers.append(w)
    states = []
    for i, kind in enumerate(cfg_block.layer_types):
        if kind == "linear_attention":
            states.append({k: v.cpu() for k, v in synth.gdn_states(cfg_block, batch, 1, seed, f"cpu.{i}", "cuda").items()})
        else:
            states.append({k: v.cpu() for k, v in synth.kv_states(cfg_block, batch, max_seq_len, [context] * batch, seed, f"cpu.{i}", "cuda").items()})
    x = synth.hidden_states((batch, 1, cfg_block.hidden_size), seed, "cpu.decode.x")
    inp = batch_step_inputs(cfg_block, [context] * batch, max_seq_len, torch.bfloat16)
    times = []
    for _ in range(2):
        started = time.perf_counter()
        om.step_decode(cfg_block, layers, states, x, inp["cos"], inp["sin"], inp["position"], inp["active"])
        times.append(time.perf_counter() - started)
        log(f"cpu decode block {times[-1]:.2f}s")
    step = times[-1] * n_blocks
    return {
        "value": batch / step,
        "unit": "tokens/s",
        "cores": threads,
        "kind": "port",
        "sample": f"one block (3 gated-delta + 1 attention layer) of the B={batch} decode at context {context} on the CPU "
        f"oracle in bf16 ({times[-1]:.2f} s after one warm-up), x{n_blocks} for 64 layers",
    }


def decode_main(args, cfg, engine, batch: int, context: int, max_seq_len: int) -> dict:
    """Decode steps of all rows, one token each, from `context` on; inputs prepared before the timed region."""
    import torch

    from qwen38_amd import synth
    from qwen38_amd.generate import batch_step_inputs
    from qwen38_amd.steps import StepGraph

    step = StepGraph(engine)
    n = args.warmup + args.steps
    embeds = synth.hidden_states((batch, 1, cfg.hidden_size), args.seed, "bench.decode", "cuda")
    inputs = []
    for i in range(n):
        raw = batch_step_inputs(cfg, [context + i] * batch, max_seq_len, torch.bfloat16)
        inputs.append({k: v.cuda() for k, v in raw.items()})
    for i in range(args.warmup):
        step(inputs_embeds=embeds, **inputs[i])
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(args.warmup, n):
        step(inputs_embeds=embeds, **inputs[i])
    end.record()
    end.synchronize()
    ms = start.elapsed_time(end) / args.steps
    log(f"decode: {ms:.3f} ms/step")
    alg = decode_bytes(cfg, batch, context + args.warmup + args.steps // 2, args.mxfp4, args.kv_fp8)
    gbs = alg / (ms / 1000.0) / 1e9
    return {
        "metric": "decode tokens/s/GPU, 64-layer one-token step, batch 64",
        "value": round(batch / (ms / 1000.0), 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": weight_dtype(args),
        "data": "synthetic: seeded random-init weights of the 27B shapes, unit-RMS states and KV",
        "config": {"workload": f"27b-64L-b64-decode-ctx{context}" + variant(args).replace(f"-ctx{context}", ""), "global_batch": batch, "tokens_per_row": 1, "context": context,
                   "parallelism": "none (one GPU)"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "algorithmic_bytes_per_step": alg},
    }


def cpu_prefill_baseline(cfg_block, max_seq_len: int, chunk: int, seed: int, n_blocks: int) -> dict:
    """The CPU oracle's prefill of one chunk on one block (bf16, all host threads), timed once after one warm-up."""
    import torch

    from oracle import model as om
    from qwen38_amd import synth
    from qwen38_amd.generate import prefill_inputs

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    layers = []
    for i in range(cfg_block.num_hidden_layers):
        prefix = f"layers.{i}."
        w = {}
        for spec in synth.layer_specs(cfg_block, i):
            v = synth.make(spec, seed, "cuda")
            w[spec.name[len(prefix):]] = om.FP8Weight(*(x.cpu() for x in v)) if isinstance(v, tuple) else v.cpu()
        layers.append(w)
    x = synth.hidden_states((1, chunk, cfg_block.hidden_size), seed, "cpu.prefill.x")
    pi = prefill_inputs(cfg_block, 0, 0, chunk, chunk, torch.bfloat16)
    times = []
    for _ in range(2):
        states = []
        for i, kind in enumerate(cfg_block.layer_types):
            if kind == "linear_attention":
                st = synth.gdn_states(cfg_block, 1, 1, seed, f"cpu.{i}", "cuda")
                states.append({k: st[k].cpu() for k in ("recurrent_state", "conv_state")})
            else:
                states.append({k: v.cpu() for k, v in synth.kv_states(cfg_block, 1, max_seq_len, [0], seed, f"cpu.{i}", "cuda").items()})
        started = time.perf_counter()
        om.step_prefill(cfg_block, layers, states, x, pi["cos"], pi["sin"], pi["slot"], pi["start"], pi["n_valid"])
        times.append(time.perf_counter() - started)
        log(f"cpu prefill block {times[-1]:.2f}s")
    return {
        "value": chunk / (times[-1] * n_blocks),
        "unit": "prompt tokens/s",
        "cores": threads,
        "kind": "port",
        "sample": f"one block (3 gated-delta + 1 attention layer) prefilling a {chunk}-token chunk from position 0 on the "
        f"CPU oracle in bf16 ({times[-1]:.2f} s after one warm-up), x{n_blocks} for 64 layers; no MTP layer",
    }


def prefill_main(args) -> dict:
    """Prompt prefill of one row: chunks of 2048 tokens from position 0, each also through the MTP layer's cache-only
    prefill, as the reference's scheduler runs a prompt (scheduler.py:110-158)."""
    import torch

    from qwen38_amd import synth
    from qwen38_amd.config import qwen38_27b_config
    from qwen38_amd.generate import mtp_prefill_inputs, prefill_inputs
    from qwen38_amd.steps import Engine, MTPStep, StepGraph

    cfg = qwen38_27b_config(16)
    batch, chunk, n_chunks, max_seq_len = 64, 2048, 2, 4096 + 64
    engine = Engine(cfg, batch, 4, max_seq_len, mtp=True, prefill_chunk=chunk, weight_format="mxfp4" if args.mxfp4 else "e4m3",
                    kv_cache_format="fp8" if args.kv_fp8 else "bf16")
    if args.kv_fp8:
        for i in [i for i, kind in enumerate(cfg.layer_types) if kind == "full_attention"] + [engine.mtp_layer]:
            engine.set_kv_scales(i, *synth.kv_scales(cfg, args.seed, f"kv.{i}", "cuda"))
    started = time.time()
    specs = synth.model_specs(cfg, mtp=True, head=True)
    weights = ((spec.name, synth.make(spec, args.seed, "cuda")) for spec in specs)
    engine.load(synth.to_mxfp4(weights) if args.mxfp4 else weights)
    log(f"model ready in {time.time() - started:.0f}s")
    step, mtp = StepGraph(engine), MTPStep(engine)
    embeds = synth.hidden_states((1, chunk, cfg.hidden_size), args.seed, "bench.prefill", "cuda")
    inputs = []
    for c in range(n_chunks):
        pi = {k: v.cuda() for k, v in prefill_inputs(cfg, 0, c * chunk, chunk, chunk, torch.bfloat16).items()}
        mi = {k: v.cuda() for k, v in mtp_prefill_inputs(cfg, 0, c * chunk, chunk, chunk, torch.bfloat16).items()}
        inputs.append((pi, mi))

    def prompt():
        for pi, mi in inputs:
            hidden = step(inputs_embeds=embeds, **pi)
            mtp(hidden=hidden, inputs_embeds=embeds, **mi)

    for _ in range(args.warmup):
        prompt()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(args.steps):
        prompt()
    end.record()
    end.synchronize()
    ms = start.elapsed_time(end) / args.steps
    tokens = chunk * n_chunks
    log(f"prefill: {ms:.2f} ms per {tokens}-token prompt")
    h, inter = cfg.hidden_size, cfg.intermediate_size
    hv, d, c = cfg.linear_num_value_heads, cfg.linear_key_head_dim, cfg.linear_conv_dim
    hq, hkv, hd = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    n_gdn = sum(1 for k in cfg.layer_types if k == "linear_attention")
    n_attn = cfg.num_hidden_layers - n_gdn
    mlp = 3 * inter * h
    per_gdn = (c + hv * d) * h + h * hv * d + mlp + 2 * hv * h  # projections, MLP, the bf16 gate projections
    per_attn = (hq * hd * 2 + 2 * hkv * hd) * h + h * hq * hd + mlp
    mtp_w = 2 * h * h + 2 * hkv * hd * h  # fc and the k/v rows (cache_chunk)
    flops = 2.0 * tokens * (n_gdn * per_gdn + n_attn * per_attn + mtp_w)
    achieved = flops / (ms / 1000.0) / 1e12
    return {
        "metric": "prefill prompt tokens/s/GPU, 64 layers + MTP cache, 4096-token prompt in 2048-token chunks",
        "value": round(tokens / (ms / 1000.0), 1),
        "unit": "prompt tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": weight_dtype(args),
        "data": "synthetic: seeded random-init weights of the 27B shapes, a synthetic prompt",
        "config": {"workload": "27b-64L-prefill-4096-chunk2048" + variant(args), "global_batch": 1, "tokens_per_row": tokens, "context": 0,
                   "parallelism": "none (one GPU)"},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 1), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / BF16_PEAK_TFLOPS, 4), "flops_per_step": flops},
        "_engine": engine,
    }


def block_main(args, index: int) -> dict:
    """BASELINE config 3 or 4 at block level: verify steps of one 27B block (3 gated-delta + 1 attention layer,
    `q38_verify`) over B rows of K tokens from a long context, each committing the step before's accepted prefixes.
    Config 3 (B=16, K=4, 32768 cached positions) is bound by HBM (the KV stream): `roofline` is the block's algorithmic
    bytes over its time. Config 4 (B=256, K=8, 4096 cached positions) is near the MFMA balance: `roofline` is the
    block's matrix work (the projections' 2 x T x weights, attention's 4 x T x Hq x context x 256, the gated-delta
    commit and reads) over its time, against the dense bf16 peak."""
    import torch

    from qwen38_amd import synth
    from qwen38_amd.config import verify_configs
    from qwen38_amd.generate import verify_inputs
    from qwen38_amd.steps import Engine

    w = verify_configs()[index]
    cfg, batch, tokens, context, max_seq_len = w.cfg, w.batch, w.tokens, w.context, w.max_seq_len
    engine = Engine(cfg, batch, tokens, max_seq_len, mtp=False, weight_format="mxfp4" if args.mxfp4 else "e4m3",
                    kv_cache_format="fp8" if args.kv_fp8 else "bf16")
    started = time.time()
    weights = ((spec.name, synth.make(spec, args.seed, "cuda")) for spec in synth.model_specs(cfg, mtp=False, head=False))
    engine.load(synth.to_mxfp4(weights) if args.mxfp4 else weights)
    from qwen38_amd.quant import encode_kv

    for i, kind in enumerate(cfg.layer_types):
        if kind == "linear_attention":
            engine.set_gdn(i, synth.gdn_states(cfg, batch, tokens, args.seed, f"state.{i}", "cuda"))
        else:
            kv = synth.kv_states(cfg, batch, max_seq_len, [context] * batch, args.seed, f"kv.{i}", "cuda")
            if args.kv_fp8:
                ks, vs = synth.kv_scales(cfg, args.seed, f"kv.{i}", "cuda")
                engine.set_kv_scales(i, ks, vs)
                kv = {"k_cache": encode_kv(kv["k_cache"], ks), "v_cache": encode_kv(kv["v_cache"], vs)}
            engine.set_kv(i, kv["k_cache"], kv["v_cache"])
            del kv
    torch.cuda.synchronize()
    log(f"config {index} block ready in {time.time() - started:.0f}s")
    x = (synth.hidden_states((batch, tokens, cfg.hidden_size), args.seed, "bench.block", "cuda").float() * 0.02).to(torch.bfloat16)
    accepted = [1 + b % tokens for b in range(batch)]  # every accepted count, as corrupted or steered drafts give
    inputs = {k: v.cuda() for k, v in verify_inputs(cfg, [context] * batch, tokens, max_seq_len, torch.bfloat16,
                                                     [True] * batch, accepted).items()}
    out = torch.empty(batch, tokens, cfg.hidden_size, dtype=torch.bfloat16, device="cuda")

    def step():
        engine.handle.verify(x, inputs["cos"], inputs["sin"], inputs["position"], inputs["active"], inputs["accepted"], out)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(args.steps):
        step()
    end.record()
    end.synchronize()
    ms = start.elapsed_time(end) / args.steps
    assert bool(torch.isfinite(out.float()).all()), "the block's output is not finite"
    t = batch * tokens
    alg = algorithmic_bytes(cfg, batch, tokens, context, args.mxfp4, args.kv_fp8)
    block_bytes = alg["weights"] + alg["state"] + alg["kv"] + alg["io"]
    h, inter = cfg.hidden_size, cfg.intermediate_size
    hv, d, c = cfg.linear_num_value_heads, cfg.linear_key_head_dim, cfg.linear_conv_dim
    hq, hkv, hd = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    n_gdn = sum(1 for k in cfg.layer_types if k == "linear_attention")
    n_attn = cfg.num_hidden_layers - n_gdn
    gemm = n_gdn * ((c + hv * d) * h + h * hv * d + 3 * inter * h) + n_attn * ((hq * hd * 2 + 2 * hkv * hd) * h + h * hq * hd + 3 * inter * h)
    flops = 2.0 * t * gemm + n_attn * 4.0 * t * hq * context * hd + n_gdn * 2.0 * batch * hv * d * d * 3 * tokens
    log(f"config {index}: {ms:.3f} ms per block step ({t} tokens)")
    if index == 3:
        gbs = block_bytes / (ms / 1000.0) / 1e9
        roof = {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                "algorithmic_bytes_per_step": block_bytes}
    else:
        tf = flops / (ms / 1000.0) / 1e12
        roof = {"bound": "mfma", "achieved": round(tf, 1), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(tf / BF16_PEAK_TFLOPS, 4), "flops_per_step": flops}
    return {
        "metric": f"verify tokens/s/GPU through one 27B block (3 gated-delta + 1 attention layer), batch {batch}, "
                  f"{tokens} tokens, context {context}",
        "value": round(t / (ms / 1000.0), 1),
        "unit": "verify tokens/s per block",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": weight_dtype(args),
        "data": "synthetic: seeded random-init weights of the 27B shapes, unit-RMS states and KV",
        "config": {"workload": f"{w.name} (BASELINE config {index})" + variant(args), "global_batch": batch,
                   "tokens_per_row": tokens, "context": context, "parallelism": "none (one GPU)"},
        "roofline": roof,
        "block_hbm": {"algorithmic_bytes_per_step": block_bytes, "achieved": round(block_bytes / (ms / 1000.0) / 1e9, 1),
                      "unit": "GB/s"},
        "block_flops_per_step": flops,
        "_engine": engine,
        "_shape": (cfg, batch, tokens, max_seq_len, context),
    }


def cpu_block_baseline(cfg, batch: int, tokens: int, max_seq_len: int, context: int, seed: int) -> dict:
    """The CPU oracle's verify step of the same block (bf16, all host threads), timed once after one warm-up."""
    import torch

    from oracle import model as om
    from qwen38_amd import synth
    from qwen38_amd.generate import verify_inputs

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    layers = []
    for i in range(cfg.num_hidden_layers):
        prefix = f"layers.{i}."
        w = {}
        for spec in synth.layer_specs(cfg, i):
            v = synth.make(spec, seed, "cuda")
            w[spec.name[len(prefix):]] = om.FP8Weight(*(x.cpu() for x in v)) if isinstance(v, tuple) else v.cpu()
        layers.append(w)
    states = []
    for i, kind in enumerate(cfg.layer_types):
        if kind == "linear_attention":
            states.append({k: v.cpu() for k, v in synth.gdn_states(cfg, batch, tokens, seed, f"cpu.{i}", "cuda").items()})
        else:
            states.append({k: v.cpu() for k, v in synth.kv_states(cfg, batch, max_seq_len, [context] * batch, seed, f"cpu.{i}", "cuda").items()})
    x = (synth.hidden_states((batch, tokens, cfg.hidden_size), seed, "cpu.block.x").float() * 0.02).to(torch.bfloat16)
    inp = verify_inputs(cfg, [context] * batch, tokens, max_seq_len, torch.bfloat16, [True] * batch,
                        [1 + b % tokens for b in range(batch)])
    times = []
    for _ in range(2):
        started = time.perf_counter()
        om.step_verify(cfg, layers, states, x, inp["cos"], inp["sin"], inp["position"], inp["active"], inp["accepted"])
        times.append(time.perf_counter() - started)
        log(f"cpu block {times[-1]:.2f}s")
    return {
        "value": batch * tokens / times[-1],
        "unit": "verify tokens/s per block",
        "cores": threads,
        "kind": "port",
        "sample": f"the same block's verify step (B={batch}, K={tokens}, context {context}) on the CPU oracle in bf16, "
        f"{times[-1]:.2f} s after one warm-up",
    }


def vendor_gemm_main(args) -> dict:
    """This build's GEMMs beside the vendor library's at the verify step's shapes: torch's bf16 matmul and FP8
    `_scaled_mm` (hipBLASLt on ROCm) against `q38_mlp_up` (the gate/up pair with SwiGLU, FP8 e4m3 weights widened to
    bf16 for the bf16 MFMA) and `q38_fp8_linear` (bf16 output) at 256 tokens, each averaged over 100 back-to-back
    launches after 10 warm-up ones. A reference point for the MFMA fractions: at 256 tokens neither reaches the dense
    peak."""
    import torch

    from qwen38_amd import ext
    from qwen38_amd.quant import quantize_e4m3

    def timeit(fn, iters=100):
        for _ in range(10):
            fn()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(iters):
            fn()
        end.record()
        end.synchronize()
        return start.elapsed_time(end) / iters * 1000.0

    g = torch.Generator(device="cuda").manual_seed(args.seed)
    rows, rows_out = 256, []
    for name, k, n in (("gate/up (SwiGLU)", 5120, 2 * 17408), ("qkvz", 5120, 16384), ("o_proj", 6144, 5120), ("down", 17408, 5120)):
        a = torch.randn(rows, k, generator=g, device="cuda").to(torch.bfloat16)
        b = torch.randn(n, k, generator=g, device="cuda").to(torch.bfloat16)
        bf = timeit(lambda: a @ b.T)
        one = torch.ones((), device="cuda")
        a8, b8 = a.to(torch.float8_e4m3fn), b.to(torch.float8_e4m3fn)
        f8 = timeit(lambda: torch._scaled_mm(a8, b8.T, scale_a=one, scale_b=one, out_dtype=torch.bfloat16))
        flop = 2.0 * rows * k * n
        entry = {"gemm": name, "tokens": rows, "k": k, "n": n, "hipblaslt_bf16_us": round(bf, 1),
                 "hipblaslt_fp8_us": round(f8, 1), "hipblaslt_bf16_tflops": round(flop / bf / 1e6, 1)}
        if name.startswith("gate") or name == "qkvz":
            coded, scales = quantize_e4m3(b.float() * 0.02)
            tiles, tscales = ext.pack_weight(coded, scales)
            scratch = ext.linear_scratch(rows, k)
            if name.startswith("gate"):
                out = torch.empty(ext.library().q38_tiles_size(rows, n // 2), dtype=torch.uint8, device="cuda")
                ext.mlp_up(a, rows, k, tiles, tscales, n // 2, scratch=scratch, out=out)
                ours = timeit(lambda: ext.mlp_up(None, rows, k, tiles, tscales, n // 2, scratch=scratch, out=out))
            else:
                ours = timeit(lambda: ext.fp8_linear(a, tiles, tscales, n, scratch=scratch))
            entry.update(this_build_us=round(ours, 1), this_build_tflops=round(flop / ours / 1e6, 1))
        rows_out.append(entry)
        log(f"{entry}")
        del a, b, a8, b8
    return {"metric": "GEMM time at the verify step's shapes, this build against hipBLASLt (torch)", "unit": "us",
            "n_gpus": 1, "data": "synthetic", "gemms": rows_out,
            "note": "this build's qkvz time includes the e5m2 activation tiles kernel; its o_proj and down projections run "
                    "split-K inside the step (see profiles/spec_step_27b_b64_k4_kernel_trace.md), not as standalone calls"}


def weight_dtype(args) -> str:
    kv = ", fp8 e4m3 KV cache" if args.kv_fp8 else ""
    mfma = (", scaled fp8 MFMA (e4m3 x e5m2) for the projections, bf16 MFMA for the head" if getattr(args, "mfma", "bf16") == "fp8"
            else ", bf16 MFMA (fp32 accumulate)")
    if args.mxfp4:
        return "mxfp4 (e2m1 + e8m0) decoder weights, fp8 e4m3 mtp/head weights" + kv + mfma
    return "fp8 e4m3 weights" + kv + mfma


def variant(args) -> str:
    ctx = f"-ctx{args.context}" if getattr(args, "context", 512) != 512 else ""
    return ("-mxfp4" if args.mxfp4 else "") + ("-kvfp8" if args.kv_fp8 else "") + ctx


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--decode", action="store_true", help="time the one-token decode graph instead of the speculative step")
    ap.add_argument("--prefill", action="store_true", help="time the prefill form (one 4096-token prompt) instead")
    ap.add_argument("--mxfp4", action="store_true", help="decoder-layer projections as MXFP4 (half the weight bytes)")
    ap.add_argument("--context", type=int, default=512,
                    help="cached positions per row before the timed steps (BASELINE's configs use 512)")
    ap.add_argument("--kv-fp8", action="store_true", help="KV caches as e4m3 bytes with per-layer scales")
    ap.add_argument("--config", type=int, choices=(3, 4), default=None,
                    help="time BASELINE config 3 (long context) or 4 (high batch, 8 tokens) at block level instead")
    ap.add_argument("--mfma", choices=("bf16", "fp8"), default="bf16",
                    help="the projections' MFMA: bf16 (default, float32-grade sums) or the scaled FP8 MFMA")
    ap.add_argument("--no-alternatives", action="store_true",
                    help="skip the extra timing of the same step with the other projection MFMA")
    ap.add_argument("--vendor-gemm", action="store_true",
                    help="time the step's GEMM shapes on hipBLASLt (torch bf16 and FP8) beside this build's GEMMs")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="first run one plain elementwise copy (bitwise_not) of MIB MiB, for counter calibration")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU: this build has no multi-GPU path (rows shard across GPUs with no exchange); "
              f"--gpus {args.gpus} is not supported", file=sys.stderr)
        return 2

    import torch

    from qwen38_amd.config import qwen38_27b_config

    batch, tokens, seed = 64, 4, args.seed
    context = args.context
    max_seq_len = max(1024, (context + 512 + 31) // 32 * 32)
    cfg = qwen38_27b_config(16)
    log(f"device {torch.cuda.get_device_name(0)}")
    if args.copy_probe:
        # A kernel of known HBM traffic (reads and writes MIB MiB once) to scale FETCH_SIZE / WRITE_SIZE counters by.
        src = torch.full((args.copy_probe << 20,), 0x5A, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        torch.bitwise_not(src, out=dst)
        torch.cuda.synchronize()
        log(f"copy probe: {args.copy_probe} MiB read and written by one bitwise_not kernel")
        del src, dst
    if args.vendor_gemm:
        print(json.dumps(vendor_gemm_main(args)), flush=True)
        return 0
    if args.config is not None:
        result = block_main(args, args.config)
        engine, shape = result.pop("_engine"), result.pop("_shape")
        if not args.no_cpu_baseline:
            del engine
            torch.cuda.empty_cache()
            result["cpu_baseline"] = cpu_block_baseline(shape[0], shape[1], shape[2], shape[3], shape[4], seed)
        print(json.dumps(result), flush=True)
        return 0
    if args.prefill:
        result = prefill_main(args)
        engine = result.pop("_engine")
        if not args.no_cpu_baseline:
            del engine
            torch.cuda.empty_cache()
            result["cpu_baseline"] = cpu_prefill_baseline(qwen38_27b_config(1), 1024, 512, seed, 16)
        print(json.dumps(result), flush=True)
        return 0
    engine, st = build(cfg, batch, tokens, max_seq_len, context, seed, args.mxfp4, args.kv_fp8, args.mfma)
    if args.decode:
        result = decode_main(args, cfg, engine, batch, context, max_seq_len)
        if not args.no_cpu_baseline:
            from qwen38_amd.config import qwen38_27b_config as big

            del engine
            torch.cuda.empty_cache()
            result["cpu_baseline"] = cpu_decode_baseline(big(1), batch, max_seq_len, context, seed, 16)
        print(json.dumps(result), flush=True)
        return 0

    def step(graph: bool = True):
        engine.handle.spec_step(st["position"], st["index"], st["match"], st["accepted"], st["active"], st["hidden"],
                                st["picks"], st["drafts"], graph=graph)

    def timed(graph: bool) -> tuple[float, int]:
        start_pos = st["position"].clone()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record()
        for _ in range(args.steps):
            step(graph)
        end.record()
        end.synchronize()
        return start.elapsed_time(end) / args.steps, int((st["position"] - start_pos).sum())

    # Warmup as launches, then the captured graph's first use for each gated-delta parity (capture + instantiate).
    for i in range(args.warmup):
        step(graph=False)
        torch.cuda.synchronize()
        log(f"warmup step {i + 1}/{args.warmup} done")
    for _ in range(2):
        step(graph=True)
    torch.cuda.synchronize()
    log("graph captured for both gated-delta parities")
    ms, accepted = timed(graph=True)
    value = accepted / (ms * args.steps / 1000.0)
    log(f"{ms:.3f} ms/step as one HIP graph per step, {accepted} accepted tokens over {args.steps} steps")
    ms_launches, _ = timed(graph=False)
    log(f"{ms_launches:.3f} ms/step as individual launches")

    # The dominant kernel inside real steps: the same number of steps again with HIP events around every gate/up GEMM
    # launch on the step's stream (64 layers + 3 MTP calls per step).
    engine.handle.kernel_timer(True)
    for _ in range(args.steps):
        step()
    launches, total_ms = engine.handle.kernel_timer(False)
    kernel_ms = total_ms / max(launches, 1)
    # Every step above records a non-finite head row or a row past its last usable position in the device's status
    # word instead of stopping; a run that hit either measures nothing, so it fails here.
    engine.handle.raise_step_errors()
    log("step status word clear after every step")
    log(f"gate/up GEMM inside the steps: {launches} launches, {kernel_ms * 1000:.1f} us each")
    flops = 2.0 * batch * tokens * 2 * cfg.intermediate_size * cfg.hidden_size
    achieved = flops / (kernel_ms / 1000.0) / 1e12
    peak = FP8_PEAK_TFLOPS if args.mfma == "fp8" else BF16_PEAK_TFLOPS
    alg = algorithmic_bytes(cfg, batch, tokens, context, args.mxfp4, args.kv_fp8)
    step_gbs = alg["total"] / (ms / 1000.0) / 1e9
    result = {
        "metric": "accepted tokens/s/GPU, 64-layer verify step, batch 64, 4 tokens; HBM GB/s %peak",
        "value": round(value, 2),
        "unit": "accepted tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "ms_per_step_launches": round(ms_launches, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": weight_dtype(args),
        "data": "synthetic: seeded random-init weights of the 27B shapes, unit-RMS states and KV",
        "config": {
            "workload": (f"27b-64L-b64-k4-ctx{context}-mtp-head" + variant(args).replace(f"-ctx{context}", "")
                         + (" (BASELINE config 2)" if context == 512 else "")),
            "global_batch": batch,
            "tokens_per_row": tokens,
            "context": context,
            "parallelism": "none (one GPU)",
        },
        "roofline": {
            "bound": "mfma",
            "kernel": f"gemm_kernel<2,4,2,2,e5m2,3,SWIGLU,{'e2m1' if args.mxfp4 else 'e4m3'},{args.mfma} MFMA,KU=2> (MLP gate/up, 256 x 34816 x 5120)",
            "achieved": round(achieved, 1),
            "peak": peak,
            "unit": "TFLOP/s",
            "frac": round(achieved / peak, 4),
            "traffic": profiled_traffic(),
            "avg_ms": round(kernel_ms, 4),
            "launches_timed": launches,
        },
        "step_roofline": {
            "bound": "hbm",
            "achieved": round(step_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(step_gbs / HBM_PEAK_GBS, 4),
            "algorithmic_bytes_per_step": alg["total"],
        },
        "accepted_per_step": accepted / args.steps,
    }
    if not args.no_alternatives and not args.decode:
        # The same step with the other projection MFMA, timed the same way on a second engine (reported beside the
        # line, not as its value: the FP8 MFMA's sums are not float32-grade).
        other = "fp8" if args.mfma == "bf16" else "bf16"
        del engine
        torch.cuda.empty_cache()
        engine, st = build(cfg, batch, tokens, max_seq_len, context, seed, args.mxfp4, args.kv_fp8, other)
        for _ in range(args.warmup):
            step(graph=False)
        for _ in range(2):
            step(graph=True)
        ms_other, acc_other = timed(graph=True)
        engine.handle.raise_step_errors()
        log(f"with the {other} MFMA: {ms_other:.3f} ms/step")
        result["alternative"] = {"projection_mfma": other, "ms_per_step": round(ms_other, 4),
                                 "value": round(acc_other / (ms_other * args.steps / 1000.0), 2),
                                 "step_hbm_frac": round(alg["total"] / (ms_other / 1000.0) / 1e9 / HBM_PEAK_GBS, 4)}
    if not args.no_cpu_baseline:
        from qwen38_amd.config import qwen38_27b_config as big

        del engine
        torch.cuda.empty_cache()
        result["cpu_baseline"] = cpu_baseline(big(1), batch, tokens, max_seq_len, context, seed, accepted / args.steps, 16)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
