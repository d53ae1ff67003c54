"""Benchmark of the Qwen3 token loop on one MI355X.

Protocol of the reference's `bench` command (src/main.rs:466-530) on seeded
synthetic weights. A "step" is one pass of the whole workload: reset the
cache, prefill the prompt (timed, logits copied to the host as the reference
writes them), take the argmax of the prefill logits (untimed, as main.rs),
then decode the workload's full token count (timed: every decode step with
its argmax, or with the device sampler for workload 5). `--steps K` runs K
timed passes after `--warmup W` untimed ones; the decode window of every
pass is the workload's own (512 tokens at KV 512 -> 1024 for the headline),
whatever K is.

`value` = decode tokens per second over the K passes (total decode tokens /
total decode time) with the weights resident in HBM. Reported alongside:
prefill tok/s, the decode step's HBM bytes and fraction of peak, the
dominant decode kernel's roofline (the fused rmsnorm + gate/up + silu*up
matvec, timed per launch inside real decode steps with HIP events bound to
the launch; its HBM traffic from the committed rocprofv3 counter summary),
the same decode window sampled with the CLI's sampling defaults on the
device sampler (greedy workloads; `sampled_decode_tok_s`), and the CPU oracle
(the C++ restatement of the reference's AVX2 path) on a bounded sample of
the same workload on the host cores.

usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload 1..5]

Workloads (4 is the default and the headline):
  1  Qwen3-0.6B Q4_K_M   48-token prompt,   32 greedy tokens
  2  Qwen3-0.6B Q8_0     48-token prompt,  128 greedy tokens (KV up to 176)
  3  Qwen3-4B  Q4_K_M   256-token prompt,  256 greedy tokens
  4  Qwen3-8B  Q4_K_M   512-token prompt,  512 greedy tokens
  5  Qwen3-32B Q4_K_M  4096-token prompt,  256 sampled tokens (temperature 0.7,
     top-k 40, top-p 0.95, repetition penalty 1.1 over the last 64, the
     CLI's fixed seed; src/main.rs:44-52)
"""
import argparse
import ctypes
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

WORKLOADS = rlh.WORKLOADS

# CPU oracle sample per workload: (prompt tokens prefilled in the default
# mode, prompt tokens prefilled with RUST_LLAMA_BATCH_INT=1, greedy decode
# tokens after the default-mode prefill), sized for roughly 10-30 s of host
# work. Where the default-mode prefill is the workload's whole prompt, the
# CPU decodes at the start of the GPU's decode window.
CPU_SAMPLE = {1: (48, 48, 32), 2: (48, 48, 128), 3: (256, 128, 64), 4: (512, 128, 32), 5: (32, 32, 8)}

METRIC = "decode tok/s, prefill tok/s, % HBM roofline"
MODEL_NAMES = {"qwen3-0.6b-q4km": "Qwen3-0.6B Q4_K_M", "qwen3-0.6b-q8_0": "Qwen3-0.6B Q8_0",
               "qwen3-4b-q4km": "Qwen3-4B Q4_K_M", "qwen3-8b-q4km": "Qwen3-8B Q4_K_M",
               "qwen3-32b-q4km": "Qwen3-32B Q4_K_M"}


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def kv_read_bytes(spec, t):
    """f32 K and V rows read by attention at context length t (all layers)."""
    return 2 * spec.n_layer * t * spec.n_head_kv * spec.head_dim * 4


def run_pass(cache, prompt, n_decode, sampled, params, never):
    """One workload pass; returns (prefill_s, decode_s, tokens)."""
    cache.reset()
    t0 = time.perf_counter()
    logits = cache.forward_into(prompt, 0)
    prefill_s = time.perf_counter() - t0
    if not sampled:
        first = cache.greedy_next()
        t1 = time.perf_counter()
        toks = cache.generate_greedy(first, n_decode)
        return prefill_s, time.perf_counter() - t1, toks
    # Model::generate's loop (model.rs:760-774): sample from the last logits,
    # append, forward the token; the sampler runs on the device and returns
    # only the token
    del logits
    P = len(prompt)
    recent = np.empty(P + n_decode, np.uint32)
    recent[:P] = prompt
    state = ctypes.c_uint64(rlh.load().rlh_sampler_init(params.seed))
    one = np.empty(1, np.uint32)
    t1 = time.perf_counter()
    for i in range(n_decode):
        tok = cache.sample_next(params, recent[:P + i], state)
        if tok == never:
            raise RuntimeError("sampled the end-of-sequence id")
        recent[P + i] = tok
        one[0] = tok
        cache.forward_into(one, P + i, copy=False)
    return prefill_s, time.perf_counter() - t1, recent[P:].copy()


def cpu_baseline(spec, tensors, prompt, n_prompt, n_prompt_int, n_decode):
    """The oracle on the host cores: prefill of n_prompt tokens in the
    reference's default mode (f32 fused products, as shipped), then n_decode
    greedy tokens in the default mode (AVX2 integer path), by the cmd_bench
    protocol; then a prefill of n_prompt_int tokens with
    RUST_LLAMA_BATCH_INT=1."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle

    lib = oracle.load()
    threads = lib.orc_get_threads()
    om = oracle.OracleModel(spec, tensors)
    oc = om.new_cache(max(n_prompt + n_decode, n_prompt_int) + 1)
    t0 = time.time()
    res_def, toks = oc.bench(prompt[:n_prompt], n_decode, oracle.MODE_DEFAULT, warmup=False)
    res_int, _ = oc.bench(prompt[:n_prompt_int], 0, oracle.MODE_BATCH_INT, warmup=False)
    wall = time.time() - t0
    oc.close()
    om.close()
    return {"decode_tok_s": res_def.generated / res_def.decode_s,
            "prefill_tok_s_default": res_def.prompt_len / res_def.prefill_s,
            "prefill_tok_s_batch_int": res_int.prompt_len / res_int.prefill_s,
            "generated": res_def.generated, "threads": threads, "wall_s": wall}


def trace_launch_us(config):
    """Average duration of the dominant kernel (k_mv<TY, 2>) over the decode
    launches of the committed rocprofv3 kernel trace of this workload
    (profiles/), or None."""
    path = os.path.join(ROOT, "profiles", f"decode_prefill_kernels_{config}_stats.txt")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("#   decode passes,") and "avg" in line:
                    return float(line.split("avg", 1)[1].split("us")[0])
    except (OSError, ValueError):
        pass
    return None


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
    ap.add_argument("--steps", type=int, default=3, help="timed passes of the whole workload")
    ap.add_argument("--warmup", type=int, default=1, help="untimed passes before them")
    ap.add_argument("--seed", type=int, default=rlh.WORKLOAD_SEED)
    ap.add_argument("--probe-steps", type=int, default=32,
                    help="decode steps whose dominant-kernel launches are timed with HIP events")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle sample")
    ap.add_argument("--prefill-only", action="store_true",
                    help="time the prefill of each pass only (no decode, no JSON line; for counter runs)")
    ap.add_argument("--kernel-launches", type=int, default=0,
                    help="with --prefill-only: then launch the dominant decode kernel (rmsnorm + gate/up "
                         "+ silu*up) this many times back to back, rotating over the layers (for counter runs)")
    ap.add_argument("--calib-copy-mb", type=int, default=0,
                    help="also run a device-to-device copy of this many MiB (counter calibration under rocprofv3)")
    args = ap.parse_args()

    if args.gpus != 1:
        print("bench.py: the benchmark runs on one GPU only (the token loop of one model on one MI355X); "
              "--gpus must be 1", file=sys.stderr)
        sys.exit(2)
    if args.steps < 1 or args.warmup < 0:
        print("bench.py: --steps must be >= 1 and --warmup >= 0", file=sys.stderr)
        sys.exit(2)

    config, n_prompt, n_decode, sampled = WORKLOADS[args.workload]
    spec = rlh.SPECS[config]
    lib = rlh.load()
    nthreads = min(16, os.cpu_count() or 1)
    t0 = time.time()
    tensors = rlh.synth_model(spec, args.seed, lib, nthreads)
    log(f"synthesised {config} in {time.time() - t0:.1f}s")
    t0 = time.time()
    model = rlh.Model(spec, tensors)
    log(f"uploaded {lib.rlh_model_weight_bytes(model.h) / 1e9:.2f} GB in {time.time() - t0:.1f}s")

    prompt = rlh.synth_tokens(args.seed + 1, n_prompt, spec.vocab)
    cache = model.new_cache(n_prompt + n_decode + 1)
    params = rlh.sampling_params()  # the CLI defaults (main.rs:44-52)
    never = spec.vocab + 7            # end-of-sequence id no token can take: fixed token counts

    if args.prefill_only:
        for i in range(args.warmup + args.steps):
            cache.reset()
            t0 = time.perf_counter()
            cache.forward_into(prompt, 0)
            log(f"prefill {i + 1}/{args.warmup + args.steps}: {n_prompt / (time.perf_counter() - t0):.1f} tok/s")
        if args.kernel_launches > 0:
            us = cache.profile_matvec(rlh.T_FFN_GATE, args.kernel_launches)
            log(f"{args.kernel_launches} back-to-back launches of the gate/up kernel: {us:.3f} us each")
        if args.calib_copy_mb > 0:
            calibration_copy(args.calib_copy_mb)
        cache.close()
        model.close()
        return
    for i in range(args.warmup):
        run_pass(cache, prompt, n_decode, sampled, params, never)
        log(f"warm-up pass {i + 1}/{args.warmup}")
    prefill_s = decode_s = 0.0
    passes = []
    tokens = None
    t_all = time.perf_counter()
    for i in range(args.steps):
        p_s, d_s, toks = run_pass(cache, prompt, n_decode, sampled, params, never)
        prefill_s += p_s
        decode_s += d_s
        passes.append(round(n_decode / d_s, 2))
        if tokens is None:
            tokens = toks
        elif not np.array_equal(tokens, toks):
            raise RuntimeError(f"pass {i} produced a different token sequence")
        log(f"pass {i + 1}/{args.steps}: prefill {n_prompt / p_s:.1f} tok/s, decode {n_decode / d_s:.2f} tok/s")
    wall_s = time.perf_counter() - t_all
    tok_s = args.steps * n_decode / decode_s
    prefill_tok_s = args.steps * n_prompt / prefill_s

    # per-token HBM traffic of the decode loop: packed weights + f32 KV read
    # at the window's average context + the K/V row written
    wbytes = spec.weight_bytes_per_token()
    t_avg = n_prompt + (n_decode + 1) / 2.0
    kvw = 2 * spec.n_layer * spec.n_head_kv * spec.head_dim * 4
    step_bytes = wbytes + kv_read_bytes(spec, t_avg) + kvw
    hbm_frac_decode = step_bytes * tok_s / (HBM_PEAK_GBS * 1e9)

    # the same window sampled (Model::generate's loop with the CLI defaults)
    sampled_tok_s = None
    if not sampled:
        _, sd_s, _ = run_pass(cache, prompt, n_decode, True, params, never)
        sampled_tok_s = round(n_decode / sd_s, 2)
        log(f"sampled decode: {sampled_tok_s} tok/s")

    # dominant decode kernel: the fused rmsnorm + ffn_gate/ffn_up + silu*up
    # launch (k_mv<TY, 2>), each launch timed with HIP events bound to it
    # inside real decode steps (36 launches per step at 8B)
    E, F = spec.n_embd, spec.n_ff
    ff_ty = spec.types[rlh.T_FFN_GATE]
    pair_bytes = (2 * F * rlh.row_bytes(ff_ty, E)  # gate + up weights
                  + 2 * E * 4                       # residual row and ffn_norm weights
                  + F * 4 + F + (F // 32) * 16)     # h (f32) and its Q8 blocks
    cache.reset()
    cache.forward_into(prompt, 0, copy=False)
    probe_steps = max(1, min(args.probe_steps, n_decode))
    mv_us, mv_launches = cache.profile_decode_kernel(rlh.T_FFN_GATE, cache.greedy_next(), probe_steps)
    mv_gbs = pair_bytes / (mv_us * 1e-6) / 1e9
    # the same kernel launched back to back (one event pair around them all,
    # rotating over every layer's weights so that they stream from HBM), and
    # its average over the decode launches of the committed kernel trace
    b2b_launches = spec.n_layer * 8
    b2b_us = cache.profile_matvec(rlh.T_FFN_GATE, b2b_launches)
    tr_us = trace_launch_us(config)
    traffic = measured_traffic(config)

    model_name = MODEL_NAMES[config]
    decode_desc = ("sampled (temperature 0.7, top-k 40, top-p 0.95, repetition penalty 1.1 over the last 64, "
                   "seed 0x123456789abcdef0)" if sampled else "greedy")
    out = {
        "metric": f"{METRIC} ({model_name}, 1 GPU)",
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1000.0 * wall_s / args.steps, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded N(0,0.02) weights quantized "
                + "/".join(sorted({rlh.TYPE_NAMES.get(t, str(t)) for t in spec.types.values()}))
                + ", norms 1+N(0,0.02), uniform random prompt ids)",
        "config": {"workload": f"{config}: {n_prompt}-token prefill then {n_decode} {decode_desc} decode tokens "
                               f"(KV {n_prompt} -> {n_prompt + n_decode}); one step = one pass of the workload",
                   "prompt_tokens": n_prompt, "decode_tokens": n_decode, "kv": "f32",
                   "eos": "ignored", "parallelism": "single GPU"},
        "decode_tok_s_per_pass": passes,
        "prefill_tok_s": round(prefill_tok_s, 1),
        "prefill_ms": round(1000.0 * prefill_s / args.steps, 3),
        "decode_ms_per_token": round(1000.0 / tok_s, 4),
        "decode_hbm_bytes_per_token": int(step_bytes),
        "decode_hbm_frac": round(hbm_frac_decode, 4),
        "prefill_int8_frac": round(spec.int8_ops_per_token() * prefill_tok_s / (INT8_PEAK_TOPS * 1e12), 5),
        "roofline": {"bound": "hbm",
                     "kernel": f"k_mv<{rlh.TYPE_NAMES.get(ff_ty, ff_ty)}, 2>: rmsnorm + ffn_gate/ffn_up "
                               f"2x{F}x{E} + silu*up",
                     "achieved": round(mv_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(mv_gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "avg_launch_us": round(mv_us, 3), "launches_timed": int(mv_launches),
                     "timing": "HIP events bound to each launch inside decode steps (about 0.9 us longer than "
                               "an unbound launch)",
                     "back_to_back_us": round(b2b_us, 3), "back_to_back_launches": b2b_launches,
                     "frac_back_to_back": round(pair_bytes / (b2b_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                     "trace_us": tr_us,
                     "frac_trace": (round(pair_bytes / (tr_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
                                    if tr_us else None),
                     "bytes_per_launch": int(pair_bytes)},
        "decode": "sampled" if sampled else "greedy",
        "sampled_decode_tok_s": sampled_tok_s,
        "tokens_head": [int(t) for t in tokens[:8]],
    }

    if args.no_cpu:
        out["cpu_baseline"] = None
    else:
        cp, ci, cd = CPU_SAMPLE[args.workload]
        r = cpu_baseline(spec, tensors, prompt, cp, ci, cd)
        out["cpu_baseline"] = {
            "value": round(r["decode_tok_s"], 3), "unit": "tok/s", "cores": r["threads"], "kind": "port",
            "prefill_tok_s_default": round(r["prefill_tok_s_default"], 2),
            "prefill_tok_s_batch_int": round(r["prefill_tok_s_batch_int"], 2),
            "sample": f"oracle (C++ restatement of the reference's AVX2 path) on {config}, {r['threads']} threads: "
                      f"{cp}-token prefill in the default mode, then {r['generated']} greedy decode tokens at "
                      f"KV {cp} -> {cp + r['generated']} (the GPU decodes KV {n_prompt} -> {n_prompt + n_decode}), "
                      f"then a {ci}-token prefill with RUST_LLAMA_BATCH_INT=1 (cmd_bench protocol; "
                      f"{r['wall_s']:.1f}s of host work)"}
        log(f"cpu oracle: decode {r['decode_tok_s']:.2f} tok/s, prefill {r['prefill_tok_s_default']:.2f} "
            f"(default) / {r['prefill_tok_s_batch_int']:.2f} (BATCH_INT) tok/s, {r['threads']} threads")

    cache.close()
    model.close()
    if args.calib_copy_mb > 0:
        calibration_copy(args.calib_copy_mb)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
