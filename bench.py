"""One DiT Euler step at 1024x1024 on one MI355X (4096 image + 256 text rows,
32 blocks, synthetic Q8_0 weights of the real 7B shape), through libexn-hip.so.

    python bench.py [--steps K] [--warmup W] [--no-cpu]

A step is one velocity pass over the image rows against the kept prompt K/V
(the reference's steps 2..8, src/cuda-dit.lisp:6-9) plus the Euler update,
with every input already in HBM.  The first call (the pass's workspace
allocated), an uncached step (the prompt rows too) and the whole 8-step loop are
reported beside it.  Prints one JSON line.

roofline: the dominant kernel (the gate_up product with SwiGLU fused) from
HIP events recorded around every 4th of its launches in the timed region (blocks
0, 4, .. 28 of each step), on the stream they run on; its algorithmic FLOPs per
launch are 2 x 4096 x 24576 x 4096.  traffic: HBM bytes per launch from rocprofv3 --pmc FETCH_SIZE /
WRITE_SIZE (profiles/), or null.

cpu_baseline: the oracle (oracle/exn_oracle.py, numpy fp32) timed on this
host for blocks 0..4 of the same cached workload, their mean x 32 blocks
(extrapolated).

vae_decode_1024sq: the VAE decoder (synthetic bf16 weights) on the 8-step loop's
final latent, 64 x 64 -> a 1024 x 1024 RGBA picture, the mean of 5 decodes.

    python bench.py --vae-only [--steps K] [--warmup W]

times the VAE decoder alone on a seeded 64 x 64 latent (K decodes after W) and
prints its own JSON line.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "ex-nihilo_amd"))

METRIC = "DiT Euler step ms @1024² (4096 img+256 txt tok), 1 GPU; % bf16 MFMA peak"
PEAK_TFLOPS = 2516.6          # MI355X dense bf16 MFMA (256 CUs x 4096 FLOP/clk x 2.4 GHz)
HBM_GBS = 8000.0
H = W = 64                    # latent 64 x 64: 4096 image rows
P = 256                       # text rows
LAYERS = 32
SEED = 2
TRAFFIC_FILE = os.path.join(REPO, "profiles", "gemm_gate_up_swiglu_1024sq_traffic.json")
PROBE_BYTES = 1 << 30         # --copy-probe 1024
VAE_FLOP = 17.03e12           # one decode of a 64 x 64 latent: every convolution and the attention's products


def gemm_flops_per_row():
    Wd, F = 4096, 12288
    return 2 * (4 * Wd * Wd + Wd * 2 * F + F * Wd)


def step_flops(cached):
    n = H * W if cached else P + H * W
    l = P + H * W
    n0 = P if cached else 0
    pairs = sum((l if g >= P else g + 1) for g in range(n0, n0 + n))
    gemm = LAYERS * n * gemm_flops_per_row()
    att = LAYERS * 4 * 128 * 32 * pairs
    return gemm, att, gemm + att


def cpu_baseline(blocks=5):
    """The oracle's cached block at the workload's shape (4096 image rows over 256 kept
    prompt rows + themselves) for blocks 0..BLOCKS-1, each timed once after its weights
    are dequantised; the step is their mean x 32 blocks."""
    sys.path.insert(0, REPO)
    from oracle import exn_oracle as xo
    rng = np.random.default_rng(0)
    wt = xo.SynthWeights(SEED, cache_bytes=6 << 30)
    n, l = H * W, P + H * W
    x = rng.normal(0, 1, (n, 4096)).astype(np.float32)
    mod = rng.normal(0, 0.05, (n, 4 * 4096)).astype(np.float32)
    cos, sin = xo.rope_tables(xo.positions(P, H, W)[P:])
    kf = np.zeros((l, 32, 128), np.float32)
    vf = np.zeros((l, 32, 128), np.float32)
    kf[:P] = rng.normal(0, 1, (P, 32, 128))
    vf[:P] = rng.normal(0, 1, (P, 32, 128))
    times = []
    for layer in range(blocks):
        for slot in ("attn.to_q.weight", "attn.to_k.weight", "attn.to_v.weight", "attn.to_out.0.weight",
                     "img_mlp.gate_up.weight", "img_mlp.out.weight", "attn.norm_q.weight", "attn.norm_k.weight"):
            wt("transformer_blocks.%d.%s" % (layer, slot))   # dequantised before the clock starts
        t0 = time.perf_counter()
        x = xo.block(wt, layer, x, mod, cos, sin, kf, vf, P, P, 0, 0)
        times.append(time.perf_counter() - t0)
    dt = float(np.mean(times))
    cores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    threads = int(os.environ.get("OPENBLAS_NUM_THREADS") or os.environ.get("OMP_NUM_THREADS") or cores)
    return {"value": round(dt * 1e3 * LAYERS, 1), "unit": "ms/step", "cores": min(cores, threads), "kind": "port",
            "sample": "blocks 0..%d of the cached 1024^2 step (4096 image rows over 4352 keys) in numpy fp32, "
                      "%.1f s of block time (%s s each), mean x 32 blocks: an extrapolated step"
                      % (blocks - 1, sum(times), "/".join("%.1f" % t for t in times))}


def traffic_from(fetch_db, write_db):
    """HBM bytes a launch of the gate_up product moves, from rocprofv3 --pmc FETCH_SIZE and
    WRITE_SIZE runs (KiB a dispatch) of `bench.py --copy-probe MIB`, each counter scaled by
    what it reads for the probe's device-to-device copy of a known size."""
    import sqlite3

    def per_kernel(db, counter):
        c = sqlite3.connect(db)
        rows = c.execute("select kernel_name, value from counters_collection where counter_name = ?",
                         (counter,)).fetchall()
        out = {}
        for name, v in rows:
            out.setdefault(name, []).append(float(v) * 1024.0)
        return out

    f, w = per_kernel(fetch_db, "FETCH_SIZE"), per_kernel(write_db, "WRITE_SIZE")
    copy = [k for k in f if "copyBuffer" in k]
    gemm = [k for k in f if "k_gemm_bt<3>" in k or "k_gemm_bt<3," in k]   # EPI_SWIGLU, any wave count
    if not copy or not gemm:
        sys.exit("bench.py: the databases hold no copy probe or no gate_up product")
    big = lambda v: max(v)                                   # the probe is the largest copy
    kc = max(copy, key=lambda k: big(f[k]))
    rf = big(f[kc]) / PROBE_BYTES
    wf = big(w[kc]) / PROBE_BYTES
    fetch = float(np.median(f[gemm[0]])) / rf
    write = float(np.median(w[gemm[0]])) / wf
    algo = 2 * (4096 * 4096 + 24576 * 4096 + 4096 * 12288)
    rec = {"kernel": "%s: gate_up + SwiGLU, 4096 x 24576 x 4096, bf16 weights" % gemm[0].split("(")[0].replace("void ", ""),
           "bytes_per_launch": round(fetch + write), "fetch_bytes": round(fetch), "write_bytes": round(write),
           "algorithmic_bytes": algo, "copy_probe_bytes": PROBE_BYTES,
           "fetch_factor": round(rf, 4), "write_factor": round(wf, 4),
           "launches": len(f[gemm[0]]),
           "commands": ["rocprofv3 --pmc FETCH_SIZE -d gpurun_out/pmc_fetch -o p -- python3 bench.py --steps 1 "
                        "--warmup 0 --no-cpu --copy-probe %d" % (PROBE_BYTES >> 20),
                        "rocprofv3 --pmc WRITE_SIZE -d gpurun_out/pmc_write -o p -- python3 bench.py --steps 1 "
                        "--warmup 0 --no-cpu --copy-probe %d" % (PROBE_BYTES >> 20),
                        "python3 bench.py --traffic-from gpurun_out/pmc_fetch/p_results.db "
                        "gpurun_out/pmc_write/p_results.db"]}
    with open(TRAFFIC_FILE, "w") as fh:
        json.dump(rec, fh, indent=1)
    print(json.dumps(rec))


def vae_only(steps, warmup):
    """The VAE decoder alone: a seeded 64 x 64 latent in HBM -> a 1024 x 1024 RGBA picture."""
    import exn_hip as X
    rng = np.random.default_rng(SEED)
    ctx = X.Context(0)
    vae = X.upload_vae(seed=SEED, ctx=ctx)
    z = X.DevBuf.of(ctx, rng.normal(0, 1, (64, H, W)).astype(np.float32))
    pic = X.DevBuf(ctx, (16 * H, 16 * W, 4), np.float32)
    for i in range(warmup):
        X.call("exn_vae_decode_dev", vae.h, z.h, H, W, pic.h)
    ctx.sync()
    t0 = time.perf_counter()
    for i in range(steps):
        X.call("exn_vae_decode_dev", vae.h, z.h, H, W, pic.h)
    ctx.sync()
    t = (time.perf_counter() - t0) / steps
    px = pic.get()
    vae_w, vae_s = vae.memory()
    vae.destroy()
    ctx.close()
    print(json.dumps({"metric": "VAE decode ms @1024² (64x64x64 latent -> 1024x1024 RGBA), 1 GPU",
                      "value": round(t * 1e3, 3), "unit": "ms/decode", "n_gpus": 1, "steps": steps,
                      "warmup": warmup, "higher_is_better": False, "dtype": "bf16", "data": "synthetic",
                      "config": {"workload": "vae-decode-64x64-latent", "weights": "bf16 synthetic", "seed": SEED},
                      "tflop": round(VAE_FLOP / 1e12, 2), "tflops": round(VAE_FLOP / t / 1e12, 1),
                      "mfma_peak_frac": round(VAE_FLOP / t / 1e12 / PEAK_TFLOPS, 4),
                      "picture_finite": bool(np.isfinite(px).all()),
                      "weights_gb": round(vae_w / 1e9, 3), "scratch_gb": round(vae_s / 1e9, 2),
                      "ref_rtx3090_ms": 1500.0}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--vae-only", action="store_true", help="time the VAE decoder alone")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="copy MIB MiB device to device after the set-up (the traffic counters' calibration)")
    ap.add_argument("--traffic-from", nargs=2, metavar=("FETCH_DB", "WRITE_DB"),
                    help="turn two rocprofv3 --pmc databases of a --copy-probe run into " + TRAFFIC_FILE)
    a = ap.parse_args()
    if a.traffic_from:
        traffic_from(*a.traffic_from)
        return
    if a.gpus != 1:
        print("bench.py: the step runs on one GPU; --gpus %d is not supported (a split of the image rows "
              "across GPUs is designed, not built)" % a.gpus, file=sys.stderr)
        sys.exit(2)
    if a.vae_only:
        vae_only(a.steps, a.warmup)
        return

    import exn_hip as X
    ctx = X.Context(0)
    d = X.Dit(ctx, LAYERS)
    t0 = time.perf_counter()
    d.synth(SEED)
    d.check()
    t1 = time.perf_counter()
    d.resident(True)
    w_bytes, _ = d.memory()
    print("bench: synthetic 7B Q8_0 DiT on the device in %.1f s, block matrices expanded to resident bf16 in %.1f s "
          "(%.1f GB of weights)" % (t1 - t0, time.perf_counter() - t1, w_bytes / 1e9), file=sys.stderr, flush=True)
    if a.copy_probe:
        src = X.DevBuf(ctx, (a.copy_probe << 20,), np.uint8)
        dst = X.DevBuf(ctx, (a.copy_probe << 20,), np.uint8)
        X.call("exn_copy", ctx.h, dst.h, src.h, a.copy_probe << 20)
        ctx.sync()
        src.free()
        dst.free()
    rng = np.random.default_rng(SEED)
    context = X.DevBuf.of(ctx, rng.normal(0, 1, (P, 4096)).astype(np.float32))
    latent = rng.normal(0, 1, (64, H, W)).astype(np.float32)
    z = X.DevBuf.of(ctx, latent)
    v = X.DevBuf(ctx, (64, H, W), np.float32)
    sig = X.TURBO_SIGMAS
    key = 7

    def step(i, k):
        s, s2 = sig[i % 8], sig[i % 8 + 1]
        X.call("exn_dit_velocity_dev", d.h, context.h, P, z.h, H, W, s, k, 0, None, 0, 0, v.h)
        X.call("exn_euler", ctx.h, 64 * H * W, z.h, v.h, np.float32(s2 - s))

    # the first call (the pass's workspace allocated), then an uncached step under the timed
    # key: the prompt rows too, their K/V kept (the cache holds one prefix, so the first
    # call's key is replaced)
    ctx.sync()
    t0 = time.perf_counter()
    step(0, key + 1)
    ctx.sync()
    t_first = time.perf_counter() - t0
    t0 = time.perf_counter()
    step(0, key)
    ctx.sync()
    t_uncached = time.perf_counter() - t0
    for i in range(a.warmup):
        step(1 + i, key)
    ctx.sync()
    # the timed steps carry HIP events around every 4th launch of the roofline kernel (blocks
    # 0, 4, .. 28 of each step): its mean launch time, measured live, at a quarter of the
    # events' cost to the step
    d.profile(True, classes=["gate_up"], every=4)
    ctx.sync()
    t0 = time.perf_counter()
    for i in range(a.steps):
        step(1 + i, key)
    ctx.sync()
    t_steps = time.perf_counter() - t0
    d.profile(False)
    gu_timed = d.profile_read()["gate_up"]
    ms = t_steps * 1e3 / a.steps
    # the per-kernel breakdown from 3 more steps with events around every launch
    BREAKDOWN = 3
    d.profile(True, every=1)
    for i in range(BREAKDOWN):
        step(1 + i, key)
    ctx.sync()
    d.profile(False)
    prof = d.profile_read()

    # the same cached step through the host-array boundary (exn_dit_velocity: the latent
    # uploaded, the velocity downloaded and transposed back, as the trio's callers pass them)
    lat_h = z.get()
    ctx_h = context.get()
    v_host = np.empty((64, H, W), np.float32)

    def host_step(i):   # the same prefix key: a cached pass over the kept prompt K/V
        X.call("exn_dit_velocity", d.h, X.ptr(ctx_h), P, X.ptr(lat_h), H, W, sig[1 + i % 7], key, 0, None, 0, 0,
               X.ptr(v_host))

    host_step(0)
    t0 = time.perf_counter()
    for i in range(3):
        host_step(i)
    t_host = (time.perf_counter() - t0) * 1e3 / 3

    # the whole 8-step loop from fresh noise (generate's loop, on the device)
    z.upload(latent)
    sg = np.array(sig, np.float64)
    ctx.sync()
    t0 = time.perf_counter()
    X.call("exn_dit_generate_dev", d.h, context.h, P, z.h, H, W, X.ptr(sg), len(sg), 0, None, 0, 0)
    ctx.sync()
    t_8 = time.perf_counter() - t0
    zf = z.get()
    finite = bool(np.isfinite(zf).all())

    # the picture: the VAE decoder (synthetic bf16 weights) on the loop's final latent,
    # 64 x 64 -> 1024 x 1024 RGBA, with the latent and the picture in HBM
    vae = X.upload_vae(seed=SEED, ctx=ctx)
    pic = X.DevBuf(ctx, (16 * H, 16 * W, 4), np.float32)
    for i in range(2):
        X.call("exn_vae_decode_dev", vae.h, z.h, H, W, pic.h)
    ctx.sync()
    VAE_REPS = 5
    t0 = time.perf_counter()
    for i in range(VAE_REPS):
        X.call("exn_vae_decode_dev", vae.h, z.h, H, W, pic.h)
    ctx.sync()
    t_vae = (time.perf_counter() - t0) / VAE_REPS
    px = pic.get()
    vae_w, vae_s = vae.memory()
    vae.destroy()

    gemm_f, att_f, tot_f = step_flops(True)
    tflops = tot_f / (ms * 1e-3) / 1e12
    gu_ms, gu_n, gu_f, gu_b = gu_timed
    gu_avg = gu_ms / max(gu_n, 1)
    achieved = (gu_f / max(gu_n, 1)) / (gu_avg * 1e-3) / 1e12 if gu_n else None
    traffic = None
    if os.path.exists(TRAFFIC_FILE):
        traffic = json.load(open(TRAFFIC_FILE)).get("bytes_per_launch")
    gemm_ms = sum(prof[c][0] for c in ("qkv", "out", "gate_up", "down"))
    gemm_flops = sum(prof[c][2] for c in ("qkv", "out", "gate_up", "down"))
    kernels = {c: {"ms_per_step": round(prof[c][0] / BREAKDOWN, 3), "launches_per_step": prof[c][1] // BREAKDOWN,
                   **({"tflops": round(prof[c][2] / (prof[c][0] * 1e-3) / 1e12, 1)} if prof[c][2] else {}),
                   **({"gbs": round(prof[c][3] / (prof[c][0] * 1e-3) / 1e9, 1)} if prof[c][3] and not prof[c][2]
                      else {})}
               for c in X.Dit.PROFILE_CLASSES if prof[c][1]}
    out = {
        "metric": METRIC, "value": round(ms, 3), "unit": "ms/step", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(ms, 3), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "dit-euler-step-1024x1024", "image_rows": H * W, "text_rows": P, "blocks": LAYERS,
                   "weights": "Q8_0 synthetic (7.0B block + 0.14B edge parameters)",
                   "step": "cached: image rows over kept prompt K/V, + Euler update", "seed": SEED},
        "tflops": round(tflops, 1), "mfma_peak_frac": round(tflops / PEAK_TFLOPS, 4),
        "step_tflop": round(tot_f / 1e12, 3),
        "gemm_tflops": round(gemm_flops / (gemm_ms * 1e-3) / 1e12, 1) if gemm_ms else None,
        "gemm_peak_frac": round(gemm_flops / (gemm_ms * 1e-3) / 1e12 / PEAK_TFLOPS, 4) if gemm_ms else None,
        "first_call_ms": round(t_first * 1e3, 2), "uncached_step_ms": round(t_uncached * 1e3, 2),
        "euler_8_steps_ms": round(t_8 * 1e3, 1),
        "host_boundary_velocity_ms": round(t_host, 3),
        "final_latent_finite": finite, "ref_rtx3090_ms_per_step": 1187.5,
        "kernels": kernels,
        "vae_decode_1024sq": {"ms": round(t_vae * 1e3, 2), "tflop": round(VAE_FLOP / 1e12, 2),
                              "tflops": round(VAE_FLOP / t_vae / 1e12, 1),
                              "mfma_peak_frac": round(VAE_FLOP / t_vae / 1e12 / PEAK_TFLOPS, 4),
                              "picture_finite": bool(np.isfinite(px).all()),
                              "weights_gb": round(vae_w / 1e9, 3), "scratch_gb": round(vae_s / 1e9, 2),
                              "ref_rtx3090_ms": 1500.0},
        "roofline": {"bound": "mfma", "kernel": "gemm gate_up + SwiGLU, 4096 x 24576 x 4096, bf16 weights (resident expansion of Q8_0)",
                     "achieved": round(achieved, 1) if achieved else None, "peak": PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_TFLOPS, 4) if achieved else None, "traffic": traffic,
                     "avg_launch_ms": round(gu_avg, 4), "launches_timed": gu_n},
    }
    if not a.no_cpu:
        print("bench: timing the CPU baseline (oracle, one block)", file=sys.stderr, flush=True)
        out["cpu_baseline"] = cpu_baseline()
    d.destroy()
    ctx.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
