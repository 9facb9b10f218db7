#!/usr/bin/env python3
"""Decode benchmark of the quantized Qwen3 hot path on one MI355X.

Workload: Qwen3-1.7B shape, Q4_K linears with Q6_K
attn_v / ffn_down / output (untied), synthetic seeded N(0, 0.02) weights;
prefill a 1024-token prompt (std::mt19937_64(42) % vocab, as
tools/bench_decode.cpp:208-213), then greedy decode at positions 1024..,
KV cache capacity 4096.

A step is one decode token: one launch of the persistent cooperative decode
kernel (embedding, 28 layers, final norm + lm_head, device argmax feeding the
next token; one workgroup per CU, stages linked by tagged dataflow words), or
the captured hipGraph of the per-stage kernels where the persistent kernel has
no instantiation.  W warm-up steps run first; then K steps are timed with host
wall clock around (sync, K launches, sync), and HIP events on the decode
stream give the GPU time per step used for the roofline.  Prints ONE JSON line.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0  # MI355X published HBM3E bandwidth

STEP_DESC = {
    "persistent": "persistent kernel, one launch per token",
    "graph": "hipGraph of the per-stage kernels, one launch per token",
    "eager": "per-stage kernels launched one by one",
}
# HBM bytes per launch of the dominant kernel from two rocprofv3 --pmc runs
# (FETCH_SIZE and WRITE_SIZE, each scaled by what the counter reads for a
# device copy of known size in the same run), with the commit they were
# measured at (re-measured whenever the persistent kernel changes):
# profiles/persist2_kernel_traffic_qwen3-1.7b-q4k.md.
MEASURED_TRAFFIC = {
    ("qwen3-1.7b-q4k", "persistent"): (1_510_464_168, "43b4e7b"),
}
KERNEL_DESC = {
    "persistent": "persist2_kernel: the whole decode step (all layers, lm_head, argmax) in one launch",
    "graph": "captured decode step (hipGraph launch)",
    "eager": "decode step (eager kernel sequence)",
}

CONFIGS = {
    # BASELINE.json configs[2]
    "qwen3-1.7b-q4k": dict(vocab=151936, hidden=2048, intermediate=6144, layers=28, n_q=16, n_kv=8, head_dim=128,
                           tied=False, embed="Q4_K", q="Q4_K", k="Q4_K", v="Q6_K", o="Q4_K", gate="Q4_K",
                           up="Q4_K", down="Q6_K", output="Q6_K", prompt=1024, decode=512, cap=4096),
    # the layout of a real Qwen3-1.7B-Q4_K_M file: tied Q6_K embedding (FP16
    # lm_head clone), attn_v / ffn_down Q6_K on llama.cpp's use_more_bits
    # layers and Q4_K elsewhere
    "qwen3-1.7b-q4k_m": dict(vocab=151936, hidden=2048, intermediate=6144, layers=28, n_q=16, n_kv=8, head_dim=128,
                             tied=True, embed="Q6_K", q="Q4_K", k="Q4_K", v="Q4_K", o="Q4_K", gate="Q4_K",
                             up="Q4_K", down="Q4_K", output="Q6_K", more_bits="Q6_K", prompt=1024, decode=512,
                             cap=4096),
    # BASELINE.json configs[1]
    "qwen3-0.6b-q8_0": dict(vocab=151936, hidden=1024, intermediate=3072, layers=28, n_q=16, n_kv=8, head_dim=128,
                            tied=True, embed="Q8_0", q="Q8_0", k="Q8_0", v="Q8_0", o="Q8_0", gate="Q8_0",
                            up="Q8_0", down="Q8_0", output="Q8_0", prompt=512, decode=256, cap=2048),
    # Mistral-Small-3.1-24B text decoder (no QK-norm, untied), Q4_K_M-style mix
    "mistral-small-3.1-24b-q4k": dict(arch="mistral3", vocab=131072, hidden=5120, intermediate=32768, layers=40,
                                      n_q=32, n_kv=8, head_dim=128, eps=1e-5, theta=1e9, context=131072,
                                      tied=False, embed="Q4_K", q="Q4_K", k="Q4_K", v="Q6_K", o="Q4_K",
                                      gate="Q4_K", up="Q4_K", down="Q6_K", output="Q6_K", prompt=1024,
                                      decode=128, cap=2048),
    # LLM2Vec's base, Meta-Llama-3-8B (no QK-norm), as a GGUF Q4_K_M-style mix
    "llama3-8b-q4k": dict(arch="mistral3", vocab=128256, hidden=4096, intermediate=14336, layers=32, n_q=32,
                          n_kv=8, head_dim=128, eps=1e-5, theta=5e5, context=8192, tied=False, embed="Q4_K",
                          q="Q4_K", k="Q4_K", v="Q6_K", o="Q4_K", gate="Q4_K", up="Q4_K", down="Q6_K",
                          output="Q6_K", prompt=1024, decode=256, cap=2048),
    # BASELINE.json configs[4]
    "qwen3-8b-q4k": dict(vocab=151936, hidden=4096, intermediate=12288, layers=36, n_q=32, n_kv=8, head_dim=128,
                         tied=False, embed="Q4_K", q="Q4_K", k="Q4_K", v="Q4_K", o="Q4_K", gate="Q4_K",
                         up="Q4_K", down="Q4_K", output="Q6_K", prompt=2048, decode=256, cap=2304),
}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def synth_path(name: str, seed: int) -> Path:
    d = Path(os.environ.get("BROLM_BENCH_DIR", "/tmp"))
    return d / f"brolm_synth_{name}_s{seed}.gguf"


def make_model_file(name: str, seed: int) -> Path:
    import brolm_amd as ba

    c = CONFIGS[name]
    path = synth_path(name, seed)
    if not path.exists():
        spec = ba.SynthSpec(**{k: v for k, v in c.items() if k not in ("arch", "prompt", "decode", "cap")}, seed=seed)
        t0 = time.time()
        tmp = path.with_suffix(".tmp")
        write = ba.write_synth_mistral3 if c.get("arch") == "mistral3" else ba.write_synth_qwen3
        write(spec, str(tmp))
        os.replace(tmp, path)
        log(f"synthetic checkpoint {path.name}: {path.stat().st_size / 1e9:.3f} GB in {time.time() - t0:.1f} s")
    return path


def cpu_baseline(path: Path, context: int, prompt: list[int], seconds: float) -> dict:
    """The oracle (C, FP32 on dequantized weights, OpenMP over the host
    cores) decoding at the GPU run's context: the KV cache is filled to the
    prompt length without a prefill (the prefill of a 1024-token prompt takes
    minutes in FP32 and is not the measured quantity), then three timed
    segments of greedy decode of about seconds / 3 each; the best segment's
    tok/s is reported, as tools/bench_decode.cpp:241-281 keeps the best of its
    repetitions."""
    import oracle

    t0 = time.time()
    m = oracle.Model(str(path))
    load_s = time.time() - t0
    max_steps = 4096
    m.allocate_cache(context + 3 * max_steps + 1)
    m.fill_cache(context, seed=7)
    tok = prompt[-1]
    best, seg_steps = 0.0, []
    for _ in range(3):
        steps, t0 = 0, time.time()
        while steps < max_steps:
            lg = m.forward([tok], last_only=True)
            tok, _ = oracle.argmax(lg[0])
            steps += 1
            if time.time() - t0 > seconds / 3:
                break
        dt = time.time() - t0
        seg_steps.append(steps)
        best = max(best, steps / dt)
    cpu = "unknown CPU"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": round(best, 3),
        "unit": "tok/s",
        "cores": oracle.num_threads(),
        "kind": "port",
        "sample": f"oracle FP32 greedy decode at context {context} (KV cache filled, no prefill), best of 3 "
                  f"segments of {seg_steps} tokens (~{seconds / 3:.0f} s each; weight dequant/load "
                  f"{load_s:.1f} s excluded); {oracle.num_threads()} OpenMP threads of {os.cpu_count()} "
                  f"visible, {cpu}",
    }


def stream_copy_gbs(torch, mib: int = 2048, reps: int = 10) -> float:
    """Device-to-device copy bandwidth (read + write bytes / time), the
    measured counterpart of the 8 TB/s denominator."""
    n = mib << 20
    src = torch.empty(n, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    gbs = 2.0 * n * reps / (e0.elapsed_time(e1) * 1e-3) / 1e9
    del src, dst
    torch.cuda.empty_cache()
    return gbs


def text_path(ba, path: Path, model, prompt: list[int]) -> dict:
    tk = ba.Tokenizer.from_gguf(str(path))
    corpus = ("The decoder reads the tokens of the prompt, 128 at a time; the sampler picks the next one. " * 12000)
    t0 = time.perf_counter()
    n_ids = len(tk.encode(corpus))
    enc_s = time.perf_counter() - t0
    model.truncate_cache(0)
    gen_opts = ba.GenerateOptions(max_new_tokens=64, sampling=ba.SamplingParams(temperature=0.0), stop_on_eos=False)
    text_prompt = tk.decode(prompt)
    ba.generate_text(model, tk, text_prompt[:2000], gen_opts)   # warm-up
    t0 = time.perf_counter()
    ba.generate_text(model, tk, text_prompt[:2000], gen_opts)
    gen_text_s = time.perf_counter() - t0
    tokenizer = {"encode_mb_s": round(len(corpus) / enc_s / 1e6, 2), "encode_ids_s": round(n_ids / enc_s),
                 "sample": f"{len(corpus) / 1e6:.2f} MB English-like text, {n_ids} ids, 1 host thread",
                 "generate_text_ms": round(gen_text_s * 1e3, 2),
                 "generate_text_note": "decoded 2000-byte prompt re-encoded, 64 greedy tokens, decode"}
    return tokenizer


def sampled_rate(ba, model, prompt, device: bool) -> float:
    """tok/s of generate() with T 0.8 / top-k 40 / top-p 0.95, 64 tokens from a
    16-token prompt (one untimed run first), the draw on the device or on the host."""
    sp = ba.SamplingParams(temperature=0.8, top_k=40, top_p=0.95, seed=1)
    opts = ba.GenerateOptions(max_new_tokens=64, sampling=sp, stop_on_eos=False, device_sampling=device)
    ba.generate(model, prompt[:16], -1, opts)
    t0 = time.perf_counter()
    n = len(ba.generate(model, prompt[:16], -1, opts))
    return round(n / (time.perf_counter() - t0), 2)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="timed decode steps (default: the config's decode)")
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--config", default="qwen3-1.7b-q4k", choices=sorted(CONFIGS))
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--cpu-seconds", type=float, default=18.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--batched-only", type=int, default=0, metavar="M",
                    help="time only the batched decode of M sequences (prompt context each) and print its "
                         "throughput (for profiler runs)")
    ap.add_argument("--sampled-only", action="store_true",
                    help="time only sampled generation with the device sampler and print its throughput "
                         "(for profiler runs)")
    ap.add_argument("--prefill-only", action="store_true",
                    help="time the prompt prefill only and print its throughput (for hardware-counter runs)")
    ap.add_argument("--decode-only", action="store_true",
                    help="prefill, then time only the greedy decode steps and print their throughput (for "
                         "profiler and hardware-counter runs)")
    ap.add_argument("--kv-cap", type=int, default=0, metavar="N",
                    help="KV cache capacity in positions (default: the config's)")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="first copy this many MiB device to device (a reference dispatch of known bytes for "
                         "hardware-counter runs)")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "multi-GPU decode is not part of this build", file=sys.stderr)
        return 2

    import brolm_amd as ba

    if args.calib_copy_mib > 0:
        import torch

        n = args.calib_copy_mib << 20
        src = torch.ones(n, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"calibration copy: {args.calib_copy_mib} MiB read + {args.calib_copy_mib} MiB written")
        del src, dst

    c = CONFIGS[args.config]
    steps = args.steps if args.steps is not None else c["decode"]
    path = make_model_file(args.config, args.seed)
    ba.init()
    mistral = c.get("arch") == "mistral3"
    if mistral:
        cfg = ba.Mistral3Config.from_gguf(str(path)).text
        model = ba.Mistral3TextModel(cfg)
    else:
        cfg = ba.Qwen3Config.from_gguf(str(path))
        model = ba.Qwen3Model(cfg)
    t0 = time.time()
    model.load_weights(str(path))
    log(f"loaded in {time.time() - t0:.1f} s")
    prompt = ba.prompt_ids(c["prompt"], cfg.vocab_size, seed=42)
    cap = max(args.kv_cap or c["cap"], c["prompt"] + args.warmup + steps + 1)
    model.allocate_cache(cap)

    if args.sampled_only:
        rate = sampled_rate(ba, model, prompt, True)
        model.close()
        ba.shutdown()
        print(json.dumps({"metric": f"sampled generate tok/s {args.config}", "value": rate, "unit": "tok/s",
                          "sampling": "T 0.8, top-k 40, top-p 0.95, device sampler", "new_tokens": 64,
                          "data": "synthetic"}), flush=True)
        return 0

    if args.batched_only > 0:
        M, n_b = args.batched_only, 32
        if not 1 <= M <= 16:
            print("bench.py: --batched-only takes 1..16 sequences", file=sys.stderr)
            return 2
        model.allocate_batch(M, len(prompt) + n_b + 8)
        for s in range(M):
            model.prefill_slot(s, prompt)
        ids, slots = [1] * M, list(range(M))
        model.time_forward_batch(ids, slots, 4)
        for s in slots:
            model.truncate_slot(s, len(prompt))
        ms = model.time_forward_batch(ids, slots, n_b)
        model.close()
        ba.shutdown()
        print(json.dumps({"metric": f"batched decode tok/s {args.config}", "value": round(M * 1e3 / ms, 1),
                          "unit": "tok/s", "rows": M, "context": len(prompt), "steps": n_b,
                          "ms_per_step": round(ms, 4), "data": "synthetic"}), flush=True)
        return 0

    # prefill (timed separately, reported as an extra field)
    t0 = time.perf_counter()
    logits = model.forward_last(prompt)
    prefill_first_s = time.perf_counter() - t0
    first = int(logits.argmax())
    t0 = time.perf_counter()
    model.truncate_cache(0)
    logits = model.forward_last(prompt)
    prefill_s = min(prefill_first_s, time.perf_counter() - t0)
    log(f"prefill {c['prompt']} tokens: {prefill_s * 1e3:.1f} ms (first pass {prefill_first_s * 1e3:.1f} ms)")
    prefill_note = ("best of two prefills of the prompt; the first pass of 512+ rows also makes the model's FP16 "
                    "copies of its layer matrices (once per model; included in prefill_first_ms)")
    if args.prefill_only:
        model.close()
        ba.shutdown()
        print(json.dumps({"metric": f"prefill tok/s {args.config}", "value": round(c["prompt"] / prefill_s, 1),
                          "unit": "tok/s", "prompt_tokens": c["prompt"], "ms": round(prefill_s * 1e3, 3),
                          "prefill_first_ms": round(prefill_first_s * 1e3, 3), "note": prefill_note,
                          "data": "synthetic"}), flush=True)
        return 0
    if args.decode_only:
        if args.warmup > 0:
            model.time_decode_steps(first, args.warmup)
        model.truncate_cache(len(prompt))
        mode = model.decode_mode()
        t0 = time.perf_counter()
        gpu_ms = model.time_decode_steps(first, steps)
        wall = time.perf_counter() - t0
        wbytes = model.decode_weight_bytes()
        model.close()
        ba.shutdown()
        print(json.dumps({"metric": f"decode tok/s bs=1 {args.config}", "value": round(steps / wall, 2),
                          "unit": "tok/s", "steps": steps, "decode_step": mode,
                          "gpu_ms_per_step_events": round(gpu_ms, 5),
                          "achieved_gbs": round(wbytes / (gpu_ms * 1e-3) / 1e9, 1), "data": "synthetic"}),
              flush=True)
        return 0
    # bidirectional encode (DenseDecoder::forward_encode, the LLM2Vec pass) of
    # the first 512 prompt tokens; the KV cache is not touched
    n_enc = min(512, len(prompt))
    model.forward_encode(prompt[:n_enc])
    t0 = time.perf_counter()
    model.forward_encode(prompt[:n_enc])
    encode_s = time.perf_counter() - t0
    log(f"encode {n_enc} tokens: {encode_s * 1e3:.1f} ms")

    # warm-up steps, then roll back to the end of the prompt
    if args.warmup > 0:
        model.time_decode_steps(first, args.warmup)
    model.truncate_cache(len(prompt))

    mode = model.decode_mode()
    log(f"decode step path: {mode}")
    # timed region: K decode steps
    t0 = time.perf_counter()
    gpu_ms = model.time_decode_steps(first, steps)
    wall = time.perf_counter() - t0
    ms_per_step = wall * 1e3 / steps
    tok_s = steps / wall

    # reference-shaped loop (forward_last + logits download + host argmax)
    model.truncate_cache(len(prompt))
    n_ref = min(64, steps)
    tok = first
    t0 = time.perf_counter()
    for _ in range(n_ref):
        tok = int(model.forward_last([tok]).argmax())
    ref_tok_s = n_ref / (time.perf_counter() - t0)

    # sampled generation (temperature 0.8, top-k 40, top-p 0.95): the draw on
    # the device (default) against the host sampler (logits download + sort)
    sampled = {("device" if dev else "host"): sampled_rate(ba, model, prompt, dev) for dev in (True, False)}

    # text path: the checkpoint's own tokenizer (host), and generate_text
    # (encode -> greedy generate -> decode) end to end; Qwen3 only (Mistral's
    # tokenizer is Tekken, not part of this build)
    tokenizer = None
    if not mistral:
        tokenizer = text_path(ba, path, model, prompt)

    # multi-sequence batched decode: M sequences, each holding the prompt in
    # its own KV slot, stepped together (one weight pass per M tokens)
    batched = {}
    n_b = 32
    model.allocate_batch(16, len(prompt) + n_b + 8)
    for s in range(16):
        model.prefill_slot(s, prompt)
    for M in (4, 16):
        slots = list(range(M))
        ids = [first] * M
        model.time_forward_batch(ids, slots, 4)
        for s in slots:
            model.truncate_slot(s, len(prompt))
        ms = model.time_forward_batch(ids, slots, n_b)
        batched[str(M)] = round(M * 1e3 / ms, 1)
        for s in slots:
            model.truncate_slot(s, len(prompt))
    log(f"batched decode tok/s: {batched}")

    import torch

    copy_gbs = stream_copy_gbs(torch)
    wbytes = model.decode_weight_bytes()
    achieved = wbytes / (gpu_ms * 1e-3) / 1e9
    kvd = cfg.num_key_value_heads * cfg.head_dim
    avg_ctx = len(prompt) + steps / 2
    kv_bytes = 2 * cfg.num_hidden_layers * avg_ctx * kvd * 2
    result = {
        "metric": ("decode tok/s bs=1 Qwen3-1.7B Q4_K; quant-GEMV HBM GB/s as % of peak"
                   if args.config == "qwen3-1.7b-q4k" else f"decode tok/s bs=1 {args.config}"),
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16 activations / Q4_K+Q6_K weights, fp32 accumulate",
        "data": "synthetic: seeded N(0,0.02) weights quantized to GGUF blocks, mt19937_64(42) prompt",
        "config": {"workload": args.config, "prompt_tokens": c["prompt"], "decode_tokens": steps, "kv_cap": cap,
                   "batch": 1, "sampling": "greedy (device argmax)", "decode_step": STEP_DESC[mode]},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": (MEASURED_TRAFFIC.get((args.config, mode)) or (None,))[0],
                     "traffic_measured_at": (MEASURED_TRAFFIC.get((args.config, mode)) or (None, None))[1],
                     "kernel": KERNEL_DESC[mode],
                     "algorithmic_bytes_per_launch": wbytes, "gpu_ms_per_launch": round(gpu_ms, 5)},
        "gpu_ms_per_step_events": round(gpu_ms, 5),
        "hbm_stream_copy_gbs": round(copy_gbs, 1),
        "roofline_frac_of_stream_copy": round(achieved / copy_gbs, 4),
        "weight_bytes_per_token": wbytes,
        "kv_bytes_per_token_avg": int(kv_bytes),
        "prefill_tok_s": round(c["prompt"] / prefill_s, 1),
        "prefill_first_ms": round(prefill_first_s * 1e3, 3),
        "prefill_note": prefill_note,
        "encode_tok_s": round(n_enc / encode_s, 1),
        "sampled_tok_s": sampled,
        "sampled_note": "generate, 64 tokens, T 0.8 / top-k 40 / top-p 0.95: device sampler vs host sampler",
        "encode_note": f"forward_encode of {n_enc} tokens (bidirectional, cacheless, hidden states downloaded)",
        "ref_loop_tok_s": round(ref_tok_s, 2),
        "batched_decode_tok_s": batched,
        "batched_decode_note": (f"forward_batch over M sequences of {len(prompt)}-token context each, {n_b} "
                                "steps, wall clock, logits left on the device; key = M"),
        "tokenizer": tokenizer,
    }
    # every device buffer and the op stream go before the process exit path (a
    # profiler wrapping this run finalizes there)
    model.close()
    ba.shutdown()
    if mistral and not args.no_cpu_baseline:
        log("cpu baseline skipped: the FP32 oracle of a 24B model needs ~96 GB of host memory")
    elif not args.no_cpu_baseline:
        log("cpu baseline (oracle) ...")
        result["cpu_baseline"] = cpu_baseline(path, len(prompt), prompt, args.cpu_seconds)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
