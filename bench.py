#!/usr/bin/env python3
"""Throughput of the vkllm LLaMA-2 token loop on one MI355X.

Workloads (--config; the default is the headline one):
  7b       LLaMA-2-7B-shaped decoder (dim 4096, 32 layers, 32 heads of 128, FFN 11008, vocab 32000), a 128-token
           uniform-random prompt prefilled, then greedy decode at batch 1 in a 4096-position KV cache
  7b-long  the same model, a 1024-token prompt, then greedy decode to position 4095: one untimed step (its graph
           is captured then), 3070 timed (tok/s also reported near positions 1k, 2k and 4k, where attention over the
           cache grows from 4% to 13% of the bytes)
  13b      LLaMA-2-13B-shaped decoder (dim 5120, 40 layers, 40 heads of 128, FFN 13824, vocab 32000), a 2048-token
           prompt, then 127 greedy steps: two untimed, 125 timed
fp16 weights are generated on the device from seed 0 (N(0, 0.02), norm weights 1.0); prompt ids from seed 1.
Every token goes through the library's C API exactly as the reference's driver loop does
(tests/vkllm_test_infer_gguf.c:181-272): tensor_new(input, mapped) -> graph_new -> models_llama2_build_graph ->
graph_init -> upload -> graph_run -> graph_post_run -> tensor_invalid_cache -> read the arg-max id -> graph_free.
The loop runs in C (vkllm_hip_token_loop, the same API calls), so no interpreter sits between tokens.

Printed (one JSON line on stdout):
  value        decode tokens/s over exactly the timed single-token steps of that loop (host work included,
               weights and KV cache resident in HBM)
  graph_replay_tok_s  the same decode step as back-to-back replays of its captured hipGraph (device time only)
  kernels      each decode kernel's average duration over back-to-back launches between one hipEvent pair on the
               library's stream, and its algorithmic GB/s
  roofline     the dominant decode kernel (the fused RMSNorm + gate/up GEMV + SwiGLU): algorithmic bytes per
               launch / its average duration over back-to-back launches across all layers' weights
  cpu_baseline the C oracle (the CPU restatement of the reference's graph, double accumulation) timing greedy
               decode steps of the full-depth model on the host's cores (at most 16 threads)
  other_configs  (--config 7b with its own cache length, no --no-companions) the 7b-long, 13b and tiny workloads
               measured after the headline one in the same process, through the same C loop and with their own step
               counts whatever --steps says: their decode tok/s, tok/s near positions 1k/2k/4k, prefill ms, and HBM
               roofline fractions
  device_floors  the HBM read rate of a kernel that only streams bytes (at 192 MiB and 1 GiB) and the cost of one
               dependent, graph-replayed launch of an empty kernel, measured on the same GPU; and the decode step's
               bytes per second as a fraction of that read rate
  isolated_kernels  (--config 7b, no --no-isolated; alone with --isolated-only) the isolated operators through the
               public VKLLM_OP_* API: GEMV [1x4096].[4096x11008] and [1x4096].[4096x32000], GEMM
               [512x4096].[4096x4096], RMSNorm [512x4096], RoPE [1,32,512,128]; average launch duration back to back
               (operands cycled past the 256 MB memory-side cache) and the fraction of the HBM or fp16 MFMA roofline;
               also one GPU's share of the 7B decode GEMVs if they were split four ways (tensor parallel, design
               only): the column-parallel [1x4096].[4096x1024] and [1x4096].[4096x2752] and the row-parallel
               [1x1024].[1024x4096] and [1x2752].[2752x4096]
"""
import argparse
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "vkllm.c_amd"))

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, GB/s
MFMA_FP16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 matrix cores, TFLOP/s
CACHE_BYTES = 256 << 20  # MI355X memory-side cache: isolated kernels cycle through more operand bytes than this
MODEL_SEED, PROMPT_SEED = 0, 1
ATTN_SMALL_MAX = 1024  # positions up to which the decode attention is the short-cache kernel (VKLLM_ATTN_SMALL_MAX)

SHAPE_TINY = dict(n_layer=6, dim=288, n_head=6, ffn=768, vocab=32000)
SHAPE_7B = dict(n_layer=32, dim=4096, n_head=32, ffn=11008, vocab=32000)
SHAPE_13B = dict(n_layer=40, dim=5120, n_head=40, ffn=13824, vocab=32000)
CONFIGS = {
    # launch-latency bound (30 MB of weights a token): its tok/s is reported, not a roofline fraction
    "tiny": dict(shape=SHAPE_TINY, prompt=16, steps=62, warmup=2, ctx=256, name="tiny LLaMA-2 decoder (dim 288, "
                 "6 layers, 6 heads of 48, FFN 768, vocab 32000), 16-token prompt prefill then 64 greedy steps at "
                 "batch 1"),
    "7b": dict(shape=SHAPE_7B, prompt=128, steps=256, warmup=8, ctx=4096, name="LLaMA-2-7B-shaped decoder (dim 4096, "
               "32 layers, 32 heads, FFN 11008, vocab 32000), 128-token prompt prefill then greedy decode at batch 1"),
    "7b-long": dict(shape=SHAPE_7B, prompt=1024, steps=3070, warmup=1, ctx=4096, name="LLaMA-2-7B-shaped decoder, "
                    "4096-position KV cache, 1024-token prompt prefill then 3072 greedy steps at batch 1"),
    "13b": dict(shape=SHAPE_13B, prompt=2048, steps=125, warmup=2, ctx=2304, name="LLaMA-2-13B-shaped decoder "
                "(dim 5120, 40 layers, 40 heads, FFN 13824, vocab 32000), 2048-token prompt prefill then 128 greedy "
                "steps at batch 1"),
}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def decode_bytes(shape, kv):
    """Algorithmic HBM bytes of each fused decode kernel for one token at `kv` cached positions (fp16 weights
    and activations, fp32 norm weights). Each weight is read once; activations and cache rows as written."""
    D, F, V = shape["dim"], shape["ffn"], shape["vocab"]
    attn = 2 * kv * D * 2 + D * 2 + D * 2
    return {
        "fused_embed": D * 2 * 2,
        "fused_qkv_rope": 3 * D * D * 2 + D * 2 + D * 4 + D * 2 + 2 * D * 2,
        "fused_attn_small": attn,
        "fused_attn_scores": attn,
        "fused_attn_long": attn,
        "fused_o_resid": D * D * 2 + D * 2 + 2 * D * 2,
        "fused_attn_o": attn + D * D * 2 + 2 * D * 2,
        "fused_gateup": 2 * F * D * 2 + D * 2 + D * 4 + F * 2,
        "fused_down_resid": D * F * 2 + F * 2 + 2 * D * 2,
        "fused_logits": V * D * 2 + D * 2 + D * 4 + V * 2,
        "fused_argmax": V * 2 + 4,
    }


def decode_families(shape, kv):
    """The kernel families a decode step at `kv` positions runs with the library's defaults and this process's
    VKLLM_* switches: the one-kernel short-cache attention (kv <= ATTN_SMALL_MAX; with Wo in the same launch under
    VKLLM_ATTN_O=1), or the long-cache attention (one launch, or scores + P.V under VKLLM_ATTN_LONG=0)."""
    env = os.environ.get
    small_max = int(env("VKLLM_ATTN_SMALL_MAX", str(ATTN_SMALL_MAX)))
    fam = ["fused_embed", "fused_qkv_rope", "fused_gateup", "fused_down_resid", "fused_logits"]
    if env("VKLLM_ARGMAX_EPI", "1") == "0":  # else the arg max runs in the vocabulary product's launch
        fam.append("fused_argmax")
    if kv <= small_max:
        return fam + (["fused_attn_o"] if env("VKLLM_ATTN_O", "0") == "1" else ["fused_attn_small", "fused_o_resid"])
    if env("VKLLM_ATTN_LONG", "1") == "0":
        return fam + ["fused_attn_scores", "fused_attn_pv", "fused_o_resid"]
    return fam + ["fused_attn_long", "fused_o_resid"]


def step_bytes(shape, kv):
    """Whole decode step at `kv` positions: the per-layer kernels times the depth, plus embed, logits, arg max."""
    b = decode_bytes(shape, kv)
    per_layer = sum(b[k] for k in ("fused_qkv_rope", "fused_attn_scores", "fused_o_resid", "fused_gateup",
                                   "fused_down_resid"))
    argmax = b["fused_argmax"] if "fused_argmax" in decode_families(shape, kv) else 0
    return per_layer * shape["n_layer"] + b["fused_embed"] + b["fused_logits"] + argmax


def read_traffic(kernel, tag):
    """HBM bytes per launch of `kernel` measured with rocprofv3 FETCH_SIZE/WRITE_SIZE, from the committed
    summary profiles/<kernel>_<tag>_pmc.txt (line 'traffic_bytes_per_launch: N'); None when absent."""
    path = os.path.join(HERE, "profiles", f"{kernel}_{tag}_pmc.txt")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def copy_calibration(ctx, vk, mib):
    """Runs the library's COPY op (contiguous fp16, `mib` MiB read and written) 4 times: a kernel of known HBM
    traffic against which rocprofv3's FETCH_SIZE / WRITE_SIZE counters are scaled."""
    n = mib * (1 << 20) // 2
    src = ctx.tensor_from(np.zeros(n, dtype=np.float16).reshape(1, 1, 1, n), name="calib_src")
    dst = ctx.tensor([1, 1, 1, n], vk.F16, "calib_dst", vk.OP_COPY, [src])
    for _ in range(4):
        vk.check("copy", ctx.run_op("copy", dst))
    ctx.free(dst)
    ctx.free(src)
    log(f"copy calibration: 4 copies of {mib} MiB")


def oracle_threads():
    """Threads the oracle's parallel loops use (its rule: ORACLE_THREADS, else the online CPUs, at most 16)."""
    n = int(os.environ.get("ORACLE_THREADS", "0") or 0) or (os.cpu_count() or 1)
    return max(1, min(16, n))


def cpu_baseline(shape, seconds):
    """Decode tokens/s of the C oracle (the CPU restatement of the reference's graph: fp16 storage, double
    accumulation) at the workload's full depth on the host's cores. The model is built first (not timed); the sample
    is greedy decode steps from an empty cache until `seconds` have passed (attention over a short cache is under 1%
    of a step's work at these widths, so the cache length does not change the rate)."""
    sys.path.insert(0, os.path.join(HERE, "oracle"))
    import oracle_ffi as oracle

    D, F, V, L = shape["dim"], shape["ffn"], shape["vocab"], shape["n_layer"]
    t_build = time.perf_counter()
    cfg = oracle.make_cfg(L, D, shape["n_head"], F, vocab=V, ctx=64)
    m = oracle.Model(cfg=cfg, seed=MODEL_SEED)
    t_build = time.perf_counter() - t_build
    try:
        tok = [int(oracle.prompt_tokens(PROMPT_SEED, 1, V)[0])]
        n, t0 = 0, time.perf_counter()
        while True:
            ids, _, _ = m.step(tok, n)
            tok = [int(ids[-1])]
            n += 1
            el = time.perf_counter() - t0
            if (el >= seconds and n >= 2) or n >= 60:
                break
    finally:
        m.close()
    cores = oracle_threads()
    return {
        "value": round(n / el, 4),
        "unit": "tok/s",
        "cores": cores,
        "kind": "port",
        "sample": f"{n} greedy decode steps of the full {L}-layer dim-{D}/FFN-{F}/vocab-{V} model (positions 0-{n - 1}) "
                  f"in {el:.1f} s on {cores} host threads; model built from seed {MODEL_SEED} in {t_build:.0f} s "
                  f"(not timed)",
    }


def device_floors(ctx):
    """What this GPU does with kernels that do nothing else (vkllm_hip_probe_stream_read / _launch_gap): the HBM read
    rate of a kernel that only streams bytes (non-temporal 16-byte loads, each byte once, windows of a 1 GiB buffer so
    none is found in the 256 MB memory-side cache), at a decode product's size (192 MiB, gate/up is 172 MiB) and at
    1 GiB; and the time per launch of a graph-replayed chain of empty kernels (one workgroup, and 1024), the cost of
    one kernel boundary of the decode step."""
    out = {}
    for mib in (192, 1024):
        med, best = ctx.probe_stream_read(mib << 20, 16)
        out[f"stream_read_{mib}MiB"] = {"median_GBps": round(med, 1), "best_GBps": round(best, 1),
                                         "frac_of_peak": round(med / HBM_PEAK_GBS, 4)}
        log(f"  stream read of {mib} MiB windows: median {med:.0f} GB/s, best {best:.0f} GB/s")
    for blocks in (1, 1024):
        us = ctx.probe_launch_gap(256, blocks)
        out[f"launch_gap_us_{blocks}wg"] = round(us, 3)
        log(f"  dependent launch of an empty kernel ({blocks} workgroups), graph-replayed: {us:.2f} us")
    return out


def isolated_kernels(ctx, vk, reps=64):
    """The isolated-operator workload (fp16 operands, fp32 accumulation, N(0,1) inputs from fixed seeds), each run
    through the library's public VKLLM_OP_* API (tensor_new + the op) and timed as back-to-back launches between one
    hipEvent pair (vkllm_hip_time_ops). Every operator cycles through enough copies of its operands that no launch
    finds them in the GPU's 256 MB memory-side cache. Returns {name: row} with the average launch duration and the
    fraction of the roofline that bounds it (HBM for the GEMVs, RMSNorm and RoPE; fp16 MFMA for the GEMM)."""
    rng = np.random.default_rng(20)
    K = 4096
    out = {}

    def timed(name, tensors, reps_, work, unit):
        ns = ctx.time_ops(tensors, reps_) / reps_
        if unit == "TFLOP/s":
            achieved, peak = work / ns / 1e3, MFMA_FP16_PEAK_TFLOPS
            row = {"avg_us": round(ns / 1e3, 3), "flops": work, "achieved": round(achieved, 1), "unit": unit,
                   "bound": "mfma", "peak": peak}
        else:
            achieved, peak = work / ns, HBM_PEAK_GBS
            row = {"avg_us": round(ns / 1e3, 3), "bytes": work, "achieved": round(achieved, 1), "unit": unit,
                   "bound": "hbm", "peak": peak}
        row["frac"] = round(achieved / peak, 4)
        row["operand_copies"] = len(tensors)
        out[name] = row
        log(f"  isolated {name:24s} {ns / 1e3:9.2f} us  {achieved:9.1f} {unit}  {row['frac']:.3f} of peak")

    def normal(shape, dtype=np.float16):
        return rng.standard_normal(shape, dtype=np.float32).astype(dtype)

    keep = []
    try:
        # GEMV [1 x Kx] . [Kx x N] (B stored [N, Kx], the reference's mat_mul_vec case): the 7B widths, then one
        # GPU's share of the decode GEMVs split four ways (Wq/Wk/Wv and up/gate by output rows, Wo and down by input
        # columns)
        for name, N, Kx in (("gemv_1x4096x11008", 11008, K), ("gemv_1x4096x32000", 32000, K),
                            ("tp4_gemv_1x4096x1024", 1024, K), ("tp4_gemv_1x4096x2752", 2752, K),
                            ("tp4_gemv_1x1024x4096", 4096, 1024), ("tp4_gemv_1x2752x4096", 4096, 2752)):
            x = ctx.tensor_from(normal((1, 1, 1, Kx)), "x")
            keep.append(x)
            w = normal((1, 1, N, Kx))
            copies = max(1, -(-2 * CACHE_BYTES // w.nbytes))
            ops = []
            for c in range(copies):
                tw = ctx.tensor_from(w, f"w{c}")
                to = ctx.tensor([1, 1, 1, N], vk.F16, f"y{c}", vk.OP_MATMUL, [x, tw], vk.MatmulParams(1.0, 0))
                keep += [tw, to]
                ops.append(to)
            del w
            timed(name, ops, reps, N * Kx * 2 + Kx * 2 + N * 2, "GB/s")
            for t in reversed(keep):
                ctx.free(t)
            keep = []
        # GEMM [512 x 4096] . [4096 x 4096] (B stored [N, K]): matrix-core bound
        M, N = 512, 4096
        ta = ctx.tensor_from(normal((1, 1, M, K)), "a")
        tb = ctx.tensor_from(normal((1, 1, N, K)), "b")
        tc = ctx.tensor([1, 1, M, N], vk.F16, "c", vk.OP_MATMUL, [ta, tb], vk.MatmulParams(1.0, 0))
        keep += [ta, tb, tc]
        timed(f"gemm_{M}x{K}x{N}", [tc], 32, 2 * M * N * K, "TFLOP/s")
        # RMSNorm over [512 x 4096] (fp16 rows, fp32 weight 1.0) and RoPE over [1, 32, 512, 128] at offset 0
        xn = normal((1, 1, 512, K))
        wn = np.ones((1, 1, 1, K), np.float32)
        xr = normal((1, 32, 512, 128))
        for name, arr, make, nbytes in (
                ("rmsnorm_512x4096", xn,
                 lambda t, w_, c: ctx.tensor([1, 1, 512, K], vk.F16, f"n{c}", vk.OP_RMSNORM, [t, w_],
                                             vk.RmsnormParams(2.0, 1e-5)), 2 * xn.nbytes + wn.nbytes),
                ("rope_512x32x128", xr,
                 lambda t, w_, c: ctx.tensor([1, 32, 512, 128], vk.F16, f"r{c}", vk.OP_ROPE, [t],
                                             vk.RopeParams(0, 10000.0, False)), 2 * xr.nbytes)):
            copies = -(-2 * CACHE_BYTES // nbytes)
            tw = ctx.tensor_from(wn, "norm_w")
            keep.append(tw)
            ops = []
            for c in range(copies):
                ti = ctx.tensor_from(arr, f"in{c}")
                to = make(ti, tw, c)
                keep += [ti, to]
                ops.append(to)
            timed(name, ops, 4 * copies, nbytes, "GB/s")
    finally:
        for t in keep:
            ctx.free(t)
    return out


def run_workload(ctx, vk, model, shape, prompt_len, steps, warmup, prefill_reps, timing_steps):
    """Prefill and greedy decode of one workload through the C token loop (vkllm_hip_token_loop, the reference
    driver's per-token sequence): prompt steps timed one by one, then `steps` decode steps in one timed loop."""
    prompt = vk.prompt_tokens(PROMPT_SEED, prompt_len, shape["vocab"])

    # prefill: one untimed, then timed repetitions of the same prompt step at offset 0, each through the C token
    # loop (one step: tensor_new, graph_new, build_graph, init, upload, run, post_run, free)
    model.loop(prompt, 1)
    prefill_ns = []
    for _ in range(prefill_reps):
        _, sns, _ = model.loop(prompt, 1)
        prefill_ns.append(int(sns[0]))
    prefill_s = float(np.median(prefill_ns)) / 1e9
    log(f"prefill {prompt_len} tokens: {prefill_s * 1e3:.2f} ms (median of {prefill_reps})")

    # decode: prefill + warmup steps untimed, then exactly `steps` single-token steps in one C loop
    ids, _, _ = model.loop(prompt, 1 + warmup)
    pos0 = prompt_len + warmup
    ctx.sync()
    t0 = time.perf_counter()
    ids, step_ns, phase_ns = model.loop([int(ids[-1])], steps, offset=pos0)
    ctx.sync()
    decode_s = time.perf_counter() - t0
    pos = pos0 + steps
    tps = steps / decode_s
    host = {k: round(float(v) / max(steps - 1, 1) / 1e3, 2)
            for k, v in zip(("build_us", "init_upload_us", "run_us", "free_us"), phase_ns)}
    log(f"decode: {steps} steps in {decode_s:.3f} s = {tps:.1f} tok/s; per step {host}")
    at_positions = {}
    for target in (1024, 2048, 4096):
        # the 64 timed steps ending at the target position (or the first 64 when the timed steps start at most 8
        # positions past it, behind the untimed warmup steps), from the per-step wall times
        if steps < 64 or not pos0 - 8 <= target <= pos + 1:
            continue
        lo = min(max(0, target - pos0 - 64), steps - 64)
        at_positions[str(target)] = round(64 / (float(np.sum(step_ns[lo:lo + 64])) / 1e9), 1)
    if at_positions:
        log(f"decode tok/s near positions: {at_positions}")

    # device time per token: replays of the captured decode graph, back to back, no host work in between
    # (not available when graph replay is switched off, e.g. VKLLM_GRAPH=0 under a kernel tracer)
    replay_ns = None
    if os.environ.get("VKLLM_GRAPH", "1") != "0" and timing_steps > 0:
        replay_ns = model.time_kernel("decode_step", timing_steps)
        log(f"decode graph replay: {replay_ns / 1e3:.1f} us per token = {1e9 / replay_ns:.1f} tok/s")
    return dict(prefill_s=prefill_s, decode_s=decode_s, tps=tps, pos0=pos0, pos=pos, host=host,
                at_positions=at_positions, replay_ns=replay_ns)


def companion(ctx, vk, name, model, prefill_reps, timing_steps):
    """Another workload measured in the same run, on `model` when given (same shape and cache length), else on a
    model generated for it: prefill and decode as above, without per-kernel timing or a CPU baseline."""
    conf = CONFIGS[name]
    shape = conf["shape"]
    own = model is None
    if own:
        log(f"generating the {name} model on the device")
        cfg = vk.llama_config(shape["n_layer"], shape["dim"], shape["n_head"], shape["ffn"], shape["vocab"],
                              conf["ctx"])
        model = vk.Model(ctx, config=cfg, seed=MODEL_SEED)
    try:
        log(f"{name}:")
        w = run_workload(ctx, vk, model, shape, conf["prompt"], conf["steps"], conf["warmup"], prefill_reps,
                         timing_steps)
    finally:
        if own:
            model.close()
    ms = w["decode_s"] / conf["steps"] * 1e3
    mean_step_bytes = step_bytes(shape, w["pos0"] + conf["steps"] // 2 + 1)
    return {
        "workload": conf["name"],
        "decode_tok_s": round(w["tps"], 2),
        "steps": conf["steps"],
        "warmup": conf["warmup"],
        "ms_per_step": round(ms, 4),
        "decode_positions": [w["pos0"], w["pos"]],
        "decode_hbm_roofline_frac": round(mean_step_bytes / (ms / 1e3) / 1e9 / HBM_PEAK_GBS, 4),
        "decode_tok_s_near_position": w["at_positions"] or None,
        "graph_replay_tok_s_at_last_position": round(1e9 / w["replay_ns"], 1) if w["replay_ns"] else None,
        "prefill_ms": round(w["prefill_s"] * 1e3, 3),
        "prefill_tok_s": round(conf["prompt"] / w["prefill_s"], 1),
    }


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--config", choices=sorted(CONFIGS), default="7b")
    ap.add_argument("--steps", type=int, default=None, help="timed decode steps (default: the workload's)")
    ap.add_argument("--warmup", type=int, default=None, help="untimed decode steps before the timed ones")
    ap.add_argument("--prefill-reps", type=int, default=4, help="timed prompt prefills")
    ap.add_argument("--timing-steps", type=int, default=32, help="graph replays timed for the device-only rate")
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="CPU baseline sample length (0: skip)")
    ap.add_argument("--ctx", type=int, default=None, help="KV cache positions (default: the workload's)")
    ap.add_argument("--no-companions", action="store_true",
                    help="skip the 7b-long and 13b workloads that the default run also measures")
    ap.add_argument("--no-isolated", action="store_true",
                    help="skip the isolated-operator workload that runs with --config 7b")
    ap.add_argument("--isolated-only", action="store_true",
                    help="run only the isolated-operator workload (GEMVs, GEMM, RMSNorm, RoPE) and print its line")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="first run the COPY op on MIB MiB (reference kernel for rocprofv3 byte counters)")
    args = ap.parse_args()
    conf = CONFIGS[args.config]
    shape = conf["shape"]
    steps = conf["steps"] if args.steps is None else args.steps
    warmup = conf["warmup"] if args.warmup is None else args.warmup
    ctx_len = conf["ctx"] if args.ctx is None else args.ctx
    prompt_len = conf["prompt"]
    L = shape["n_layer"]

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py runs on one GPU: the token loop of this library is single-device (asked for "
              f"--gpus {args.gpus}, WORLD_SIZE {world})", file=sys.stderr)
        sys.exit(2)
    need = prompt_len + warmup + steps + 1
    if need > ctx_len:
        sys.exit(f"--ctx {ctx_len} is smaller than the {need} positions the run uses")

    os.environ.setdefault("VKLLM_QUIET", "1")
    import pyvkllm as vk

    ctx = vk.Ctx(0)
    if args.isolated_only:
        log(f"device {ctx.arch()}; isolated operators")
        iso = isolated_kernels(ctx, vk)
        floors = device_floors(ctx)
        ctx.close()
        print(json.dumps({"metric": "isolated operator kernels, fp16 operands, fp32 accumulation", "n_gpus": 1,
                          "dtype": "f16 storage, f32 accumulate", "data": "synthetic: N(0,1) operands, fixed seeds",
                          "isolated_kernels": iso, "device_floors": floors}), flush=True)
        return
    if args.copy_calibration > 0:
        copy_calibration(ctx, vk, args.copy_calibration)
    log(f"device {ctx.arch()}; generating the {args.config} model on the device")
    cfg = vk.llama_config(L, shape["dim"], shape["n_head"], shape["ffn"], shape["vocab"], ctx_len)
    model = vk.Model(ctx, config=cfg, seed=MODEL_SEED)
    w = run_workload(ctx, vk, model, shape, prompt_len, steps, warmup, args.prefill_reps, args.timing_steps)
    prefill_s, decode_s, tps, pos0, pos = w["prefill_s"], w["decode_s"], w["tps"], w["pos0"], w["pos"]
    host, at_positions, replay_ns = w["host"], w["at_positions"], w["replay_ns"]

    # per-kernel durations: back-to-back launches between one hipEvent pair on the library's stream
    nbytes = decode_bytes(shape, pos)
    used = decode_families(shape, pos)
    kernels = {}
    step_kernel_ns = 0.0
    for name in ("fused_embed", "fused_qkv_rope", "fused_attn_o", "fused_attn_small",
                 "fused_attn_long", "fused_attn_scores", "fused_attn_pv", "fused_o_resid", "fused_gateup",
                 "fused_down_resid", "fused_logits", "fused_argmax"):
        per_layer = name not in ("fused_embed", "fused_logits", "fused_argmax")
        reps = 4 * L if per_layer else 32
        try:  # kernels outside the step's variant are timed where the library takes this cache length
            avg_ns = model.time_kernel(name, reps)
        except vk.VkllmError:
            if name in used:
                raise
            continue
        if name in used:
            step_kernel_ns += avg_ns * (L if per_layer else 1)
        row = {"avg_us": round(avg_ns / 1e3, 3), "in_step": name in used}
        if name in nbytes:
            row["GBps"] = round(nbytes[name] / avg_ns, 1)
        kernels[name] = row
        log(f"  {name:20s} avg {avg_ns / 1e3:9.2f} us  {row.get('GBps', ''):>8}  {'step' if name in used else ''}")
    dom = "fused_gateup"
    dom_avg_ns = kernels[dom]["avg_us"] * 1e3
    achieved = nbytes[dom] / dom_avg_ns  # GB/s
    # bytes of the average timed step: the cache length at the middle of the timed steps
    mean_step_bytes = step_bytes(shape, pos0 + steps // 2 + 1)
    traffic = read_traffic(dom, "7b") if shape is SHAPE_7B else None

    result = {
        "metric": "decode tok/s + % HBM roofline, LLaMA-2-7B-shape fp16 bs=1; prefill tok/s",
        "value": round(tps, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(decode_s / steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 storage, f32 accumulate",
        "data": "synthetic: device-generated random-init weights (seed 0), uniform-random prompt ids (seed 1)",
        "config": {"workload": conf["name"], "name": args.config, "prompt": prompt_len,
                   "decode_positions": [pos0, pos], "kv_cache_positions": ctx_len},
        "prefill_tok_s": round(prompt_len / prefill_s, 1),
        "prefill_ms": round(prefill_s * 1e3, 3),
        "decode_hbm_roofline_frac": round(mean_step_bytes / (decode_s / steps) / 1e9 / HBM_PEAK_GBS, 4),
        "decode_bytes_per_token": mean_step_bytes,
        "decode_tok_s_near_position": at_positions or None,
        "kernel_ms_per_step": round(step_kernel_ns / 1e6, 4),
        "graph_replay_ms_per_step": round(replay_ns / 1e6, 4) if replay_ns else None,
        "graph_replay_tok_s": round(1e9 / replay_ns, 1) if replay_ns else None,
        "host_per_step": host,
        "roofline": {"kernel": dom, "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "algorithmic_bytes": nbytes[dom], "avg_us": round(dom_avg_ns / 1e3, 3)},
        "kernels": kernels,
    }
    # the other two workloads, in the default run only: 7b-long on the same model (same shape, 4096-position
    # cache), then 13b on a model of its own once the 7B one is freed
    others = None
    if not args.no_companions and args.config == "7b" and args.ctx is None:
        others = {}
        for name in ("7b-long", "13b", "tiny"):
            if name == "13b":
                model.close()
                model = None
            try:
                others[name] = companion(ctx, vk, name, model, args.prefill_reps, args.timing_steps)
            except vk.VkllmError as e:
                others[name] = {"error": str(e)}
    if model is not None:
        model.close()
    result["other_configs"] = others
    # the isolated operators (GEMVs at the 7B widths, the 512-token GEMM, RMSNorm, RoPE) through the public op API
    result["isolated_kernels"] = None
    if not args.no_isolated and args.config == "7b":
        result["isolated_kernels"] = isolated_kernels(ctx, vk)
    # the device's streaming-read rate and kernel-boundary cost, against which the decode step is read as well
    floors = device_floors(ctx)
    floors["decode_step_frac_of_stream_read_1024MiB"] = round(
        mean_step_bytes / (decode_s / steps) / 1e9 / floors["stream_read_1024MiB"]["median_GBps"], 4)
    result["device_floors"] = floors
    ctx.close()
    if args.cpu_seconds > 0:
        log(f"cpu baseline (oracle, full depth, {oracle_threads()} threads)")
        result["cpu_baseline"] = cpu_baseline(shape, args.cpu_seconds)
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
