"""Benchmark of the Qwen3 token loop on one MI355X.

Workload (default): Qwen3-8B shape, Q4_K_M mix, seeded synthetic weights;
512-token random prompt (batched prefill), then greedy decode. Protocol of
the reference's `bench` command (src/main.rs:466-530): warm-up prefill,
reset, timed prefill, timed greedy decode loop (argmax after every step,
here fused on the device). A "step" is one decode token; `value` is decode
tokens per second. Prefill tok/s, the per-token HBM roofline and the
dominant kernel's roofline are reported alongside, plus the CPU reference
(oracle) timed on a bounded sample of the same workload.

usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload 1..5]

Workloads (the five benchmark configurations; 4 is the default and the
headline):
  1  Qwen3-0.6B Q4_K_M   48-token prompt,   32 greedy tokens
  2  Qwen3-0.6B Q8_0     48-token prompt,  128 greedy tokens (KV up to 176)
  3  Qwen3-4B  Q4_K_M   256-token prompt,  256 greedy tokens
  4  Qwen3-8B  Q4_K_M   512-token prompt,  512 greedy tokens
  5  Qwen3-32B Q4_K_M  4096-token prompt,  256 sampled tokens (temperature 0.7,
     top-k 40, top-p 0.95, repetition penalty 1.1 over the last 64, the
     CLI's fixed seed; src/main.rs:44-52)
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "llama.rs_amd"))

import rlh  # noqa: E402

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, published
INT8_PEAK_TOPS = 5000.0  # MI355X dense int8, published


# workload -> (model, prompt tokens, decode tokens, sampled)
WORKLOADS = {
    1: ("qwen3-0.6b-q4km", 48, 32, False),
    2: ("qwen3-0.6b-q8_0", 48, 128, False),
    3: ("qwen3-4b-q4km", 256, 256, False),
    4: ("qwen3-8b-q4km", 512, 512, False),
    5: ("qwen3-32b-q4km", 4096, 256, True),
}


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def kv_read_bytes(spec, t):
    """f32 K and V rows read by attention at context length t (all layers)."""
    return 2 * spec.n_layer * t * spec.n_head_kv * spec.head_dim * 4


def cpu_baseline(spec, tensors, prompt, n_decode, threads):
    """The oracle (C++ restatement of the reference AVX2 path) on the host
    cores: default modes as the reference ships them. Bounded sample: a
    short prefill then n_decode timed greedy steps."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle

    lib = oracle.load()
    lib.orc_set_threads(threads)
    om = oracle.OracleModel(spec, tensors)
    oc = om.new_cache(len(prompt) + n_decode + 1)
    res, toks = oc.bench(prompt, n_decode, oracle.MODE_DEFAULT, warmup=False)
    oc.close()
    om.close()
    return res, toks


def measured_traffic(config):
    """HBM bytes per launch of the dominant kernel from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary (profiles/), or None."""
    path = os.path.join(ROOT, "profiles", f"k_mv_pair_{config}_pmc.txt")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(float(line.split(":", 1)[1]))
    except OSError:
        pass
    return None


def calibration_copy(mb):
    """A device-to-device copy of `mb` MiB (the runtime's copy kernel): the
    known-size reference for scaling the HBM byte counters."""
    import ctypes

    hip = ctypes.CDLL("libamdhip64.so")
    n = mb << 20
    a, b = ctypes.c_void_p(), ctypes.c_void_p()
    if hip.hipMalloc(ctypes.byref(a), ctypes.c_size_t(n)) or hip.hipMalloc(ctypes.byref(b), ctypes.c_size_t(n)):
        raise RuntimeError("hipMalloc for the calibration copy failed")
    for _ in range(3):
        if hip.hipMemcpy(b, a, ctypes.c_size_t(n), 3):  # hipMemcpyDeviceToDevice
            raise RuntimeError("calibration copy failed")
    hip.hipDeviceSynchronize()
    hip.hipFree(a)
    hip.hipFree(b)
    log(f"calibration copy: 3 x {mb} MiB device to device")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--workload", type=int, default=4, choices=sorted(WORKLOADS))
    ap.add_argument("--steps", type=int, default=None, help="timed decode tokens (default: the workload's)")
    ap.add_argument("--warmup", type=int, default=16, help="untimed decode tokens after the warm-up prefill")
    ap.add_argument("--config", default=None, help="model shape (default: the workload's)")
    ap.add_argument("--prompt", type=int, default=None, help="prompt tokens (default: the workload's)")
    ap.add_argument("--seed", type=int, default=20260)
    ap.add_argument("--cpu-decode", type=int, default=6, help="CPU baseline decode tokens (0 = skip)")
    ap.add_argument("--cpu-prompt", type=int, default=8, help="CPU baseline prompt tokens")
    ap.add_argument("--calib-copy-mb", type=int, default=0,
                    help="also run a device-to-device copy of this many MiB (counter calibration under rocprofv3)")
    args = ap.parse_args()

    if args.gpus != 1:
        print("bench.py: the benchmark runs on one GPU only (the token loop of one model on one MI355X); "
              "--gpus must be 1", file=sys.stderr)
        sys.exit(2)

    wl_config, wl_prompt, wl_steps, sampled = WORKLOADS[args.workload]
    args.config = args.config or wl_config
    args.prompt = args.prompt or wl_prompt
    args.steps = args.steps or wl_steps
    spec = rlh.SPECS[args.config]
    lib = rlh.load()
    nthreads = min(16, os.cpu_count() or 1)
    t0 = time.time()
    tensors = rlh.synth_model(spec, args.seed, lib, nthreads)
    log(f"synthesised {args.config} in {time.time() - t0:.1f}s")
    t0 = time.time()
    model = rlh.Model(spec, tensors)
    log(f"uploaded {lib.rlh_model_weight_bytes(model.h) / 1e9:.2f} GB in {time.time() - t0:.1f}s")

    prompt = rlh.synth_tokens(args.seed + 1, args.prompt, spec.vocab)
    max_ctx = args.prompt + max(args.steps, args.warmup) + 8
    cache = model.new_cache(max_ctx)

    params = rlh.sampling_params()  # the CLI defaults (main.rs:44-52)
    never = spec.vocab + 7            # EOS id no token can take: fixed token counts
    # warm-up: prefill + a few decode steps (pages in code, graphs, caches)
    logits = cache.forward_into(prompt, 0)
    first = cache.greedy_next()
    if args.warmup:
        cache.generate_greedy(first, args.warmup)
    if sampled and args.warmup:
        cache.reset()
        cache.generate(prompt, args.warmup, params, never)
    cache.reset()

    # timed prefill
    t0 = time.perf_counter()
    logits = cache.forward_into(prompt, 0)
    prefill_s = time.perf_counter() - t0
    first = cache.greedy_next()

    if sampled:
        # Model::generate (prefill, then sample / forward_one per token, the
        # sampler on the host): decode time = its time minus the prefill's
        cache.reset()
        t0 = time.perf_counter()
        toks = cache.generate(prompt, args.steps, params, never)
        decode_s = time.perf_counter() - t0 - prefill_s
        if len(toks) != args.steps:
            raise RuntimeError(f"generate returned {len(toks)} tokens, expected {args.steps}")
    else:
        # timed decode: exactly K steps (generate_greedy returns after the
        # device finished and the tokens were copied back)
        t0 = time.perf_counter()
        toks = cache.generate_greedy(first, args.steps)
        decode_s = time.perf_counter() - t0
    tok_s = args.steps / decode_s
    prefill_tok_s = args.prompt / prefill_s

    # per-token HBM traffic of the decode loop: packed weights + f32 KV read
    # at the average context + K/V write
    wbytes = spec.weight_bytes_per_token()
    t_avg = args.prompt + (args.steps + 1) / 2.0
    kvw = 2 * spec.n_layer * spec.n_head_kv * spec.head_dim * 4
    step_bytes = wbytes + kv_read_bytes(spec, t_avg) + kvw
    hbm_frac_decode = step_bytes * tok_s / (HBM_PEAK_GBS * 1e9)

    # dominant decode kernel: the fused rmsnorm + ffn_gate/ffn_up + silu*up
    # launch (k_mv<TY, 2>), timed per launch with HIP events on the cache's
    # stream, rotating over the layers' weights
    E, F = spec.n_embd, spec.n_ff
    ff_ty = spec.types[rlh.T_FFN_GATE]
    pair_bytes = (2 * F * rlh.row_bytes(ff_ty, E)  # gate + up weights
                  + 2 * E * 4                       # residual row and ffn_norm weights
                  + F * 4 + F + (F // 32) * 16)     # h (f32) and its Q8 blocks
    mv_us = cache.profile_matvec(rlh.T_FFN_GATE, 4 * spec.n_layer)
    mv_gbs = pair_bytes / (mv_us * 1e-6) / 1e9
    traffic = measured_traffic(args.config)

    out = {
        "metric": ("decode tok/s (Qwen3-8B Q4_K_M, 1 GPU); prefill tok/s and % HBM roofline reported alongside"
                   if args.workload == 4 else
                   f"decode tok/s ({args.config}, 1 GPU); prefill tok/s and % HBM roofline reported alongside"),
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1000.0 / tok_s, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded N(0,0.02) weights quantized "
                + "/".join(sorted({rlh.TYPE_NAMES.get(t, str(t)) for t in spec.types.values()}))
                + ", uniform random prompt ids)",
        "config": {"workload": f"{args.config}: {args.prompt}-token prefill then {args.steps} "
                               f"{'sampled (temperature 0.7, top-k 40, top-p 0.95, repetition penalty 1.1)' if sampled else 'greedy'}"
                               f" decode tokens (KV up to {args.prompt + args.steps})",
                   "prompt_tokens": args.prompt, "decode_tokens": args.steps, "kv": "f32",
                   "eos": "ignored", "parallelism": "single GPU"},
        "prefill_tok_s": round(prefill_tok_s, 1),
        "prefill_ms": round(prefill_s * 1000, 3),
        "decode_hbm_bytes_per_token": int(step_bytes),
        "decode_hbm_frac": round(hbm_frac_decode, 4),
        "prefill_int8_frac": round(spec.int8_ops_per_token() * args.prompt / prefill_s / (INT8_PEAK_TOPS * 1e12), 5),
        "roofline": {"bound": "hbm",
                     "kernel": f"k_mv<{rlh.TYPE_NAMES.get(ff_ty, ff_ty)}, pair>: rmsnorm + ffn_gate/ffn_up "
                               f"2x{F}x{E} + silu*up",
                     "achieved": round(mv_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(mv_gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "avg_launch_us": round(mv_us, 3), "bytes_per_launch": int(pair_bytes)},
        "decode": "sampled" if sampled else "greedy",
        "tokens_head": [int(t) for t in toks[:8]],
    }

    if args.cpu_decode > 0:
        cpu_prompt = prompt[: args.cpu_prompt]
        res, ctoks = cpu_baseline(spec, tensors, cpu_prompt, args.cpu_decode, nthreads)
        out["cpu_baseline"] = {"value": round(res.generated / res.decode_s, 3), "unit": "tok/s", "cores": nthreads,
                               "kind": "port",
                               "sample": f"oracle (C++ AVX2 restatement of the reference) on {args.config}: "
                                         f"{len(cpu_prompt)}-token prefill then {res.generated} greedy decode "
                                         f"tokens; prefill {res.prompt_len / res.prefill_s:.2f} tok/s"}
    else:
        out["cpu_baseline"] = None

    cache.close()
    model.close()
    if args.calib_copy_mb > 0:
        calibration_copy(args.calib_copy_mb)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
