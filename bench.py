"""Decode throughput of the 7B-shape Q4_K_M model at batch 1 on one MI355X.

One step = one greedy decode token (the whole LLaMA-like step: 32 layers +
LM head + argmax) with weights and KV cache resident in HBM.  The prompt is
processed first on the device (batched MFMA prefill: a `--prefill`-token
prefill from position 0 is timed and reported with its MFMA utilisation, then
the rest of the prompt), so the timed decode steps run at context position
`--ctx`.  Prints one JSON line.

  python bench.py [--steps K] [--warmup W] [--ctx T] [--prefill P] [--config mistral7b]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "gemv_gate_up_q4k_mistral7b_traffic.md")
GEMV_SOURCE = os.path.join(ROOT, "dotllm_amd", "csrc", "gemv.hip")


def gemv_source_hash() -> str:
    import hashlib
    with open(GEMV_SOURCE, "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()[:16]


def measured_traffic(config: str):
    """HBM bytes per gate/up launch from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE summary (counters cannot be read inside a normal run), with the
    reason when there is none.  The summary names the gemv.hip it measured
    (`gemv_source_sha256:`); a figure from another build of the kernel is
    refused rather than reported."""
    if config != "mistral7b" or not os.path.exists(TRAFFIC_PROFILE):
        return None, "no counter profile for this workload"
    fields = {}
    for line in open(TRAFFIC_PROFILE):
        if ":" in line and not line.startswith((" ", "|", "#", "`")):
            k, v = line.split(":", 1)
            fields[k.strip()] = v.strip()
    cur = gemv_source_hash()
    if fields.get("gemv_source_sha256") != cur:
        return None, (f"stale: the profile measured gemv.hip {fields.get('gemv_source_sha256', '?')}, "
                      f"this build is {cur}")
    return float(fields["traffic_bytes_per_launch"]), f"rocprofv3 FETCH_SIZE + WRITE_SIZE of gemv.hip {cur}"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_baseline(img, ctx: int, steps: int, threads: int, warmup: bool = True) -> dict:
    """The reference CPU path (oracle restatement) on the same weights; with
    threads = 1 the reference's own execution model (no Parallel, Thread or
    Task in its src/)."""
    from oracle import oracle as O
    O.set_threads(threads)
    m = O.Model(img, kv_fp16=False, context=ctx + steps + 2)
    m.kv_fill_random(ctx, seed=3)
    tok = 1
    if warmup:
        m.process_token(tok, ctx)        # warm-up step
    t0 = time.perf_counter()
    for i in range(steps):
        lg = m.process_token(tok, ctx + 1 + i)
        tok = int(lg.argmax())
    dt = time.perf_counter() - t0
    m.close()
    return {"value": steps / dt, "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"{'1 warm-up + ' if warmup else ''}{steps} greedy decode step(s) of the same model at position {ctx}+ "
                      f"(KV filled synthetically), oracle restatement, {threads} OpenMP threads of "
                      f"{os.cpu_count()} host cores"}


MFMA_PEAK_TFLOPS = 2500.0   # MI355X dense fp16/bf16 MFMA


def prefill_flops(spec: dict, n: int) -> float:
    """Algorithmic FLOPs of an n-token prompt: 2 x projection parameters x n,
    causal attention 2 hd n^2 per head and layer (QK^T + PV over the lower
    triangle), and the LM head once (the last token)."""
    d, f, L = spec["hidden"], spec["ffn"], spec["layers"]
    q, kv = spec["heads"] * spec["head_dim"], spec["kv_heads"] * spec["head_dim"]
    params = L * (2 * d * q + 2 * d * kv + 3 * d * f)
    attn = 2.0 * spec["head_dim"] * n * n * spec["heads"] * L
    return 2.0 * params * n + attn + 2.0 * d * spec["vocab"]


# The other full-size workloads, measured after the headline run: name ->
# (model, prompt tokens, KV format).  Decode is timed from the end of the prompt.
EXTRA = {"c3": ("llama1b", 512, True), "c5": ("phi3mini", 2048, True)}
# weight mixes of the synthetic models, as named in the workload label
MIX_LABELS = {"q4_k_m": "Q4_K_M", "q5_k_m": "Q5_K_M", "q8_0": "Q8_0", "phi3": "Q6_K/Q8_0"}


def extra_config(be, key: str, seed: int, steps: int) -> dict:
    """Prefill of the workload's prompt (batched MFMA path, HIP events) and the
    greedy decode loop right after it, for one of EXTRA's shapes."""
    from dotllm_amd import synth
    from dotllm_amd.engine import InferenceEngine, LoadedModel
    name, n, kv16 = EXTRA[key]
    spec = synth.SPECS[name]
    ctx = n + steps + 16
    img = synth.build_image(name, seed=seed, context=ctx)
    eng = InferenceEngine(LoadedModel.load(img), be, kv_fp16=kv16, context=ctx)
    try:
        prompt = synth.prompt(spec["vocab"], n, seed=7)
        eng.time_prefill(prompt[:min(256, n)], 0)   # warm-up
        pf_ms = eng.time_prefill(prompt, 0)
        _, tok = eng.prefill(prompt, 0)
        r = eng.time_decode(tok, n, steps)
        dec = 1000.0 * steps / r["total_ms"]
        fl = prefill_flops(spec, n)
        return {"workload": f"{name}-shape {MIX_LABELS.get(spec['mix'], spec['mix'])}, {n}-token prompt then greedy decode, batch 1, "
                            f"{'fp16' if kv16 else 'fp32'} KV",
                "prefill_tokens": n, "prefill_ms": round(pf_ms, 3), "prefill_tok_s": round(n / (pf_ms * 1e-3), 1),
                "prefill_mfma_util": round(fl / (pf_ms * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS, 4),
                "decode_tok_s": round(dec, 2), "decode_from_position": n, "decode_steps": steps,
                "decode_step_gbps": round(eng.step_bytes(n + steps // 2) * dec / 1e9, 1)}
    finally:
        eng.dispose()


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--ctx", type=int, default=4096)
    ap.add_argument("--config", default="mistral7b")
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--cpu-steps", type=int, default=2,
                    help="timed oracle steps of the single-thread baseline, after one warm-up step (about 22 s "
                         "each at the 7B shape)")
    ap.add_argument("--cpu-threads", type=int, default=0,
                    help="threads of the second, parallel oracle figure (0: up to 16)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--kernel-steps", type=int, default=8)
    ap.add_argument("--contexts", default="512,2048",
                    help="extra decode contexts timed after the main run (decode_by_context)")
    ap.add_argument("--prefill", type=int, default=2048,
                    help="tokens of the timed prefill from position 0 (0: none)")
    ap.add_argument("--synthetic-kv", action="store_true",
                    help="fill the KV cache of the first --ctx positions with random values instead of "
                         "processing a --ctx-token prompt (same decode-step work; for short profiling runs)")
    ap.add_argument("--extra", default="c3,c5",
                    help="other full-size workloads timed after the headline run (prefill + decode); '' for none")
    ap.add_argument("--eager", action="store_true",
                    help="launch the step kernel by kernel instead of replaying the captured HIP graph "
                         "(the committed rocprofv3 summaries are of eager runs, one record per kernel)")
    args = ap.parse_args()
    if args.eager:
        os.environ["LLMDOT_HIP_NO_GRAPH"] = "1"
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); the decode path is a single-GPU "
              f"batch-1 loop and no multi-GPU figure is produced.", file=sys.stderr)
        return 2

    from dotllm_amd import synth
    from dotllm_amd.backend import HipBackend
    from dotllm_amd.engine import InferenceEngine, LoadedModel

    spec = synth.SPECS[args.config]
    ffn_type = {v: k.upper() for k, v in synth.QUANT_NAMES.items()}[synth.tensor_type(spec["mix"], "blk.0.ffn_gate.weight")]
    mix_label = MIX_LABELS.get(spec["mix"], spec["mix"])
    total_ctx = args.ctx + args.warmup + 2 * args.steps + args.kernel_steps + 8
    t0 = time.perf_counter()
    img = synth.build_image(args.config, seed=args.seed, context=total_ctx)
    log(f"synthesised {args.config} image: {img.nbytes / 1e9:.2f} GB in {time.perf_counter() - t0:.1f}s")
    model = LoadedModel.load(img)
    be = HipBackend(0)
    info = be.device_info()
    t0 = time.perf_counter()
    eng = InferenceEngine(model, be, kv_fp16=True, context=total_ctx)
    log(f"uploaded weights + built step graph in {time.perf_counter() - t0:.1f}s on {info['name']} ({info['arch']})")

    prompt = synth.prompt(spec["vocab"], max(args.ctx, args.prefill), seed=7)
    pf = None
    n_pf = min(args.prefill, args.ctx) if not args.synthetic_kv else args.prefill
    if n_pf > 0:
        eng.time_prefill(prompt[:min(256, n_pf)], 0)           # warm-up (kernel loads)
        pf_ms = eng.time_prefill(prompt[:n_pf], 0)
        fl = prefill_flops(spec, n_pf)
        pf = {"tokens": n_pf, "ms": round(pf_ms, 3), "tok_s": round(n_pf / (pf_ms * 1e-3), 1),
              "flops": fl, "tflops": round(fl / (pf_ms * 1e-3) / 1e12, 1), "peak_tflops": MFMA_PEAK_TFLOPS,
              "mfma_util": round(fl / (pf_ms * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS, 4),
              "arith": "fp16 MFMA, activations as two fp16 planes (fp32-equivalent), fp32 accumulation"}
        log(f"prefill {n_pf} tokens: {pf_ms:.2f} ms, {pf['tok_s']:.0f} tok/s, {pf['tflops']:.0f} TFLOP/s "
            f"({100 * pf['mfma_util']:.1f}% of {MFMA_PEAK_TFLOPS:.0f})")
    if args.synthetic_kv:
        eng.kv_fill_random(args.ctx, seed=3)
        tok = 1
        log(f"filled {args.ctx} KV positions with random values")
    else:
        t0 = time.perf_counter()
        # the timed prefill left positions 0 .. n_pf-1 in the cache; the rest of the
        # prompt continues from there (its last token's argmax starts the decode)
        start = n_pf if n_pf < args.ctx else args.ctx - 1
        _, tok = eng.prefill(prompt[start:args.ctx], start)
        log(f"processed the rest of the {args.ctx}-token prompt in {time.perf_counter() - t0:.1f}s")
    pos = args.ctx

    if args.warmup > 0:
        eng.time_decode(tok, pos, args.warmup)
    # timed region: the device-side greedy loop, bracketed by stream synchronisation
    res = eng.time_decode(tok, pos + args.warmup, args.steps)
    ms_step = res["total_ms"] / args.steps
    value = 1000.0 / ms_step
    step_bytes = eng.step_bytes(pos + args.warmup + args.steps // 2)
    log(f"decode: {ms_step:.3f} ms/token, {value:.1f} tok/s, {step_bytes / ms_step / 1e6:.1f} GB/s step-level")

    # the same loop at shorter contexts (the cost depends on the position only)
    by_ctx = {}
    for c in sorted({int(v) for v in args.contexts.split(",") if v.strip()}):
        if 0 < c < pos:
            r = eng.time_decode(tok, c, args.steps)
            by_ctx[str(c)] = round(1000.0 * args.steps / r["total_ms"], 2)
    by_ctx[str(args.ctx)] = round(value, 2)
    log("decode by context: " + ", ".join(f"{c}: {v:.1f} tok/s" for c, v in by_ctx.items()))

    # dominant kernel: the fused gate/up SwiGLU GEMV, bracketed with HIP events
    kr = eng.time_decode(tok, pos + args.warmup + args.steps, args.kernel_steps, per_kernel=True)
    from dotllm_amd.measure import stream_peak_gbps
    stream = stream_peak_gbps(be, 1 << 30, 10)
    log(f"streaming probe over 1 GiB: read {stream['read']:.0f} GB/s, write {stream['write']:.0f} GB/s")
    per_launch_ms = kr["gemv_ms"] / max(kr["gemv_launches"], 1)
    per_launch_bytes = kr["gemv_bytes"] / max(kr["gemv_launches"], 1)
    achieved = per_launch_bytes / (per_launch_ms * 1e-3) / 1e9
    log(f"gate/up GEMV: {per_launch_ms * 1e3:.1f} us/launch, {per_launch_bytes / 1e6:.1f} MB, {achieved:.0f} GB/s")

    traffic, traffic_note = measured_traffic(args.config)
    if traffic is None:
        log(f"roofline.traffic: none ({traffic_note})")
    out = {
        "metric": "decode tok/s @batch 1, 7B-shape Q4_K_M; achieved HBM GB/s vs peak",
        "value": round(value, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic",
        "config": {"workload": f"{args.config}-shape {mix_label} greedy decode, batch 1, context {args.ctx}, fp16 KV",
                   "launch": "eager" if args.eager else "hip-graph",
                   "kv": "random fill" if args.synthetic_kv else "prompt processed on device",
                   "hidden": spec["hidden"], "layers": spec["layers"], "heads": spec["heads"],
                   "kv_heads": spec["kv_heads"], "head_dim": spec["head_dim"], "ffn": spec["ffn"],
                   "vocab": spec["vocab"], "context": args.ctx, "batch": 1},
        "step_hbm": {"bytes_per_token": step_bytes, "achieved_gbps": round(step_bytes / ms_step / 1e6, 1),
                     "peak_gbps": HBM_PEAK_GBPS, "frac": round(step_bytes / ms_step / 1e6 / HBM_PEAK_GBPS, 4)},
        "roofline": {"bound": "hbm",
                     "kernel": f"gemv_kernel<{ffn_type}, SWIGLU, RmsNorm> (ffn gate+up, {spec['ffn']}x{spec['hidden']} x2)",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic, "traffic_source": traffic_note,
                     "bytes_per_launch": per_launch_bytes, "us_per_launch": round(per_launch_ms * 1e3, 2),
                     "stream_probe_gbps": {k: round(v, 1) for k, v in stream.items()}},
        "decode_by_context": by_ctx,
        "prefill": pf,
        "cpu_baseline": None,
    }
    eng.dispose()
    extra = {}
    for key in [k.strip() for k in args.extra.split(",") if k.strip()]:
        t0 = time.perf_counter()
        extra[key] = extra_config(be, key, args.seed, args.steps)
        log(f"{key}: prefill {extra[key]['prefill_tok_s']:.0f} tok/s, decode {extra[key]['decode_tok_s']:.1f} tok/s "
            f"({time.perf_counter() - t0:.1f}s)")
    out["other_workloads"] = extra or None
    be.dispose()
    if not args.no_cpu_baseline:
        # the faithful figure: one thread, as the reference runs
        t0 = time.perf_counter()
        out["cpu_baseline"] = cpu_baseline(img, args.ctx, args.cpu_steps, 1, warmup=True)
        log(f"cpu baseline (1 thread): {out['cpu_baseline']['value']:.4f} tok/s ({time.perf_counter() - t0:.1f}s)")
        threads = args.cpu_threads or min(16, os.cpu_count() or 1)
        if threads > 1:
            t0 = time.perf_counter()
            par = cpu_baseline(img, args.ctx, 6, threads)
            out["cpu_baseline"]["parallel"] = par
            log(f"cpu baseline ({threads} threads): {par['value']:.3f} tok/s ({time.perf_counter() - t0:.1f}s)")
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
