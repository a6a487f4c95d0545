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
(extrapolated); beside it the single-block workload (1024 image + 64 text rows,
uncached) as the median of 3, and the host's CPU model, cores and BLAS.

w8a8: the same cached step in the reference's default int8 mode (exn_dit_w8a8:
activations quantised to Q8_0 by blocks of 32, int8 products), with its breakdown.

q8_0: the same cached step with the block matrices multiplied from Q8_0, the
codes dequantised inside the products (no resident bf16 copy), with its gate_up
roofline.  cfg3_1536x1024 / cfg4_edit: cached and uncached steps of the
1536 x 1024 workload (6144 image + 256 text rows) and of the edit workload
(512 text rows + a 64 x 64 reference picture + a 64 x 64 image: 8704 keys).

vae_decode_1024sq: the VAE decoder (synthetic bf16 weights) on the 8-step loop's
final latent, 64 x 64 -> a 1024 x 1024 RGBA picture, the mean of 5 decodes.

    python bench.py --vae-only [--steps K] [--warmup W]

times the VAE decoder alone on a seeded 64 x 64 latent (K decodes after W) and
prints its own JSON line.

prompt_encoder: the prompt encoder (Qwen3-VL-8B's text model, 36 blocks, synthetic Q8_0
weights) over a 256-token prompt, and over an edit prompt of 1100 tokens of which 1024 are a
1024 x 1024 picture's rows (merged and deepstack), each the mean of 3 calls with the inputs in
HBM; FLOPs counted with the model's 8 key/value heads (the q | k | v product's 6144 rows).

    python bench.py --encoder-only [--steps K] [--warmup W]

uncached: the 1024^2 step with the prompt's 256 rows through every block (the reference's
first step), K steps after W, its own JSON line.

    python bench.py --uncached-only [--steps K] [--warmup W]

vision_encode_1024sq: the vision tower (Qwen3-VL's ViT, synthetic fp16-valued
weights, fp32 arithmetic) on a 1024 x 1024 RGBA picture in HBM: 4096 patches
through 27 blocks and the four mergers, the mean of 3 encodes; its rate against
the dense fp32 MFMA peak (157.3 TFLOP/s).

    python bench.py --vision-only [--steps K] [--warmup W]

times the tower alone and prints its own JSON line.

pictures: whole pictures as the reference's README times them (1024 x 1024,
1536 x 1024 and an edit at 1024 x 1024 on an RTX 3090: about 11, 22 and 20 s):
the prompt encoder's states, the 8-step loop from fresh noise (its first step
uncached) and the VAE decode, plus for the edit the vision tower on the picture
to edit and its rows in the prompt, and the VAE encoder's latent of that
picture; each part timed between synchronisations, the mean of 2 pictures after
one.

vae_encode_1024sq: the VAE encoder (an edit's picture to its 64 x 64 latent) on
the decoded 1024 x 1024 picture, the mean of 5 encodes (--vae-only too).

    python bench.py --vae-encode-only [--steps K] [--warmup W]

times the encoder alone on a seeded picture and prints its own JSON line.
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
TRAFFIC_FILE_Q8 = os.path.join(REPO, "profiles", "gemm_gate_up_swiglu_q8_0_1024sq_traffic.json")
PROBE_BYTES = 1 << 30         # --copy-probe 1024
PEAK_F32_TFLOPS = 157.3      # MI355X dense fp32 MFMA
VAE_FLOP = 17.03e12           # one decode of a 64 x 64 latent: every convolution and the attention's products
VAE_ENC_FLOP = 3.1585e12      # one encode of a 1024 x 1024 picture, likewise (the first convolution at 4 channels)


def gemm_flops_per_row():
    Wd, F = 4096, 12288
    return 2 * (4 * Wd * Wd + Wd * 2 * F + F * Wd)


def step_flops(cached, nimg=H * W, ptext=P, nref=0, a=0):
    """Block products and attention of one step: the prefix is PTEXT text rows and NREF rows
    of a reference picture after the first A of them; attention counts the (query, key)
    pairs the mask leaves visible (image rows: all keys; the picture's rows: the picture and
    what is before it; text rows: causal)."""
    p = ptext + nref
    n = nimg if cached else p + nimg
    l = p + nimg
    n0 = p if cached else 0
    b0, b1 = a, a + nref
    pairs = 0
    for g in range(n0, n0 + n):
        pairs += l if g >= p else (b1 if b0 <= g < b1 else g + 1)
    gemm = LAYERS * n * gemm_flops_per_row()
    att = LAYERS * 4 * 128 * 32 * pairs
    return gemm, att, gemm + att


def host_info():
    """The host the CPU baseline ran on: model, usable cores, BLAS and its thread settings."""
    model = None
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    blas = None
    try:
        cfg = np.show_config(mode="dicts")
        b = cfg.get("Build Dependencies", {}).get("blas", {})
        blas = "%s %s" % (b.get("name", "?"), b.get("version", ""))
    except Exception:
        pass
    return {"cpu_model": model, "cpu_count": os.cpu_count(),
            "affinity": len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else None,
            "blas": blas, "OMP_NUM_THREADS": os.environ.get("OMP_NUM_THREADS"),
            "OPENBLAS_NUM_THREADS": os.environ.get("OPENBLAS_NUM_THREADS")}


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
    # the single-block workload: 1024 image rows (32 x 32) and 64 text rows, uncached, sigma 0.5
    c0, l0 = xo.synth_inputs(0, 64, 32, 32)
    b_times = []
    for r in range(4):   # one warm-up (dequantisation of block 0's weights), then the median of 3
        t0 = time.perf_counter()
        xo.forward(wt, c0, l0, 0.5, layers=1)
        b_times.append(time.perf_counter() - t0)
    cores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    threads = int(os.environ.get("OPENBLAS_NUM_THREADS") or os.environ.get("OMP_NUM_THREADS") or cores)
    return {"value": round(dt * 1e3 * LAYERS, 1), "unit": "ms/step", "cores": min(cores, threads), "kind": "port",
            "sample": "blocks 0..%d of the cached 1024^2 step (4096 image rows over 4352 keys) in numpy fp32, "
                      "%.1f s of block time (%s s each), mean x 32 blocks: an extrapolated step"
                      % (blocks - 1, sum(times), "/".join("%.1f" % t for t in times)),
            "one_block_1088_rows_ms": round(float(np.median(b_times[1:])) * 1e3, 1),
            "one_block_sample": "the single-block workload (1024 image + 64 text rows, uncached, sigma 0.5, "
                                "with the edge products and the velocity), median of 3 after a warm-up",
            "host": host_info()}


def traffic_from(fetch_db, write_db, q8=False, bf16_only=False):
    """HBM bytes a launch of the gate_up product moves, from rocprofv3 --pmc FETCH_SIZE and
    WRITE_SIZE runs (KiB a dispatch) of `bench.py --copy-probe MIB`, each counter scaled by
    what it reads for the probe's device-to-device copy of a known size.  Q8: the product on
    Q8_0 weights (`bench.py --q8-only --copy-probe MIB`), else on the resident bf16 ones."""
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
    # EPI_SWIGLU on bf16 weights, k_gemm_bt<3, 8, false>, or on Q8_0 ones over 4096 rows, k_gemm_q8_tall<3>
    gemm = [k for k in f if ("k_gemm_q8_tall<3>" in k if q8 else ("k_gemm_bt<3," in k and "false" in k))]
    if not copy or not gemm:
        sys.exit("bench.py: the databases hold no copy probe or no gate_up product")
    big = lambda v: max(v)                                   # the probe is the largest copy
    kc = max(copy, key=lambda k: big(f[k]))
    rf = big(f[kc]) / PROBE_BYTES
    wf = big(w[kc]) / PROBE_BYTES
    fetch = float(np.median(f[gemm[0]])) / rf
    write = float(np.median(w[gemm[0]])) / wf
    # X and Y in bf16 once; W in bf16 (2 bytes a weight) or Q8_0 (34 bytes a block of 32)
    algo = 2 * (4096 * 4096 + 4096 * 12288) + (24576 * 4096 * 34 // 32 if q8 else 2 * 24576 * 4096)
    run = "--q8-only " if q8 else ("--bf16-only " if bf16_only else "")
    fd, wd = os.path.relpath(os.path.dirname(os.path.abspath(fetch_db))), os.path.relpath(os.path.dirname(os.path.abspath(write_db)))
    rec = {"kernel": "%s: gate_up + SwiGLU, 4096 x 24576 x 4096, %s weights"
                     % (gemm[0].split("(")[0].replace("void ", ""), "Q8_0" if q8 else "bf16"),
           "bytes_per_launch": round(fetch + write), "fetch_bytes": round(fetch), "write_bytes": round(write),
           "algorithmic_bytes": algo, "copy_probe_bytes": PROBE_BYTES,
           "fetch_factor": round(rf, 4), "write_factor": round(wf, 4),
           "launches": len(f[gemm[0]]),
           "commands": ["rocprofv3 --pmc FETCH_SIZE -d %s -o p -- python3 bench.py %s--steps 1 "
                        "--warmup 0 --no-cpu --copy-probe %d" % (fd, run, PROBE_BYTES >> 20),
                        "rocprofv3 --pmc WRITE_SIZE -d %s -o p -- python3 bench.py %s--steps 1 "
                        "--warmup 0 --no-cpu --copy-probe %d" % (wd, run, PROBE_BYTES >> 20),
                        "python3 bench.py %s--traffic-from %s %s" % (run, os.path.relpath(fetch_db),
                                                                     os.path.relpath(write_db))]}
    with open(TRAFFIC_FILE_Q8 if q8 else TRAFFIC_FILE, "w") as fh:
        json.dump(rec, fh, indent=1)
    print(json.dumps(rec))


def pmc_summary(dbs):
    """A markdown table from rocprofv3 --pmc databases: per kernel, its dispatches, mean duration,
    the clock (GRBM_GUI_ACTIVE, summed over the 8 XCDs, over the duration) and the MFMA pipe's busy
    fraction (SQ_VALU_MFMA_BUSY_CYCLES over the 1024 SIMDs' cycles), with any other counter's mean."""
    import sqlite3
    acc = {}
    for db in dbs:
        c = sqlite3.connect(db)
        for kn, cn, v, t0, t1 in c.execute("select kernel_name, counter_name, value, start, end "
                                          "from counters_collection"):
            k = kn.split("(")[0].replace("void ", "")
            d = acc.setdefault(k, {})
            d.setdefault(cn, []).append(float(v))
            d.setdefault("_dur", []).append((t1 - t0) / 1e3)
    print("| kernel | dispatches | mean µs | GHz | MFMA busy | counters (mean a dispatch) |")
    print("|---|---:|---:|---:|---:|---|")
    for k, d in sorted(acc.items(), key=lambda kv: -sum(kv[1]["_dur"])):
        dur = float(np.mean(d["_dur"]))
        g = float(np.mean(d["GRBM_GUI_ACTIVE"])) if "GRBM_GUI_ACTIVE" in d else None
        # GRBM_GUI_ACTIVE sums the 8 XCDs' cycles; it also counts the dispatch's set-up and
        # drain, so under about 50 µs the clock and the busy fraction say little
        g = g if g and dur >= 50 else None
        clk = g / 8 / dur / 1e3 if g else None
        busy = float(np.mean(d["SQ_VALU_MFMA_BUSY_CYCLES"])) / (1024 * g / 8) if g and "SQ_VALU_MFMA_BUSY_CYCLES" in d else None
        rest = ", ".join("%s %.4g" % (cn, float(np.mean(v))) for cn, v in sorted(d.items())
                         if cn not in ("_dur", "GRBM_GUI_ACTIVE", "SQ_VALU_MFMA_BUSY_CYCLES"))
        n = len(d["_dur"]) // max(1, len([c for c in d if c != "_dur"]))
        print("| `%s` | %d | %.1f | %s | %s | %s |" % (k, n, dur, "%.2f" % clk if clk else "-",
                                                      "%.3f" % busy if busy is not None else "-", rest))


def smi_sample():
    """Socket power (W) and the 8 XCDs' GFX clocks (MHz) from one `amd-smi metric -p -c`."""
    import re
    import subprocess
    try:
        r = subprocess.run(["amd-smi", "metric", "-p", "-c", "-g", "0"], capture_output=True, text=True, timeout=20)
    except (OSError, subprocess.TimeoutExpired):
        return None, []
    pw = re.search(r"SOCKET_POWER:\s*([\d.]+)\s*W", r.stdout)
    clk = [int(c) for c in re.findall(r"GFX_\d+:\s*\n\s*CLK:\s*(\d+)\s*MHz", r.stdout)]
    return (float(pw.group(1)) if pw else None), clk


def power_run(seconds, step, ctx, z, latent, weights):
    """The cached step looped for SECONDS (8 steps from the same latent a round) while a thread
    samples amd-smi: the socket power and clocks the step runs at."""
    import threading
    idle = smi_sample()
    samples, stop = [], threading.Event()

    def sampler():
        while not stop.is_set():
            samples.append((time.perf_counter(),) + smi_sample())
            stop.wait(0.25)

    th = threading.Thread(target=sampler)
    t0 = time.perf_counter()
    th.start()
    n = 0
    while time.perf_counter() - t0 < seconds:
        z.upload(latent)
        for i in range(8):
            step(i, 7)
        n += 8
        ctx.sync()
    dt = time.perf_counter() - t0
    stop.set()
    th.join()
    late = [s for s in samples if s[0] - t0 > 1.0 and s[1] is not None]   # past the first second's ramp
    pw = [s[1] for s in late]
    clk = [c for s in late for c in s[2]]
    stat = lambda v: {"median": float(np.median(v)), "min": float(min(v)), "max": float(max(v))} if v else None
    print(json.dumps({"metric": "socket power and GFX clocks during the cached 1024² step loop, 1 GPU",
                      "weights": weights, "seconds": round(dt, 2), "steps": n,
                      "ms_per_step": round(dt / n * 1e3, 3), "samples": len(late),
                      "socket_power_w": stat(pw), "idle_socket_power_w": idle[0],
                      "gfx_clock_mhz": stat(clk), "peak_clock_mhz": 2400,
                      "source": "amd-smi metric -p -c -g 0, every 0.25 s from a thread"}), flush=True)


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
    t_enc, zf = vae_encode_time(ctx, vae, pic, steps, warmup)
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
                      "ref_rtx3090_ms": 1500.0, "vae_encode_1024sq": vae_encode_record(t_enc, zf)}), flush=True)


def vae_encode_time(ctx, vae, pic, reps, warmup):
    """The VAE encoder on the 1024 x 1024 picture PIC (in HBM) -> its 64 x 64 latent: (s an
    encode, whether every value is finite)."""
    import exn_hip as X
    z = X.DevBuf(ctx, (64, H, W), np.float32)
    for i in range(warmup):
        X.call("exn_vae_encode_dev", vae.h, pic.h, 16 * H, 16 * W, z.h)
    ctx.sync()
    t0 = time.perf_counter()
    for i in range(reps):
        X.call("exn_vae_encode_dev", vae.h, pic.h, 16 * H, 16 * W, z.h)
    ctx.sync()
    t = (time.perf_counter() - t0) / reps
    finite = bool(np.isfinite(z.get()).all())
    z.free()
    return t, finite


def vae_encode_only(steps, warmup):
    """The VAE encoder alone: a seeded 1024 x 1024 RGBA picture in HBM -> its 64 x 64 latent."""
    import exn_hip as X
    rng = np.random.default_rng(SEED)
    ctx = X.Context(0)
    vae = X.upload_vae(seed=SEED, ctx=ctx)
    pic = X.DevBuf.of(ctx, np.clip(rng.normal(0, 0.5, (16 * H, 16 * W, 4)), -1, 1).astype(np.float32))
    t, finite = vae_encode_time(ctx, vae, pic, steps, warmup)
    vae_w, vae_s = vae.memory()
    vae.destroy()
    ctx.close()
    rec = vae_encode_record(t, finite)
    print(json.dumps(dict({"metric": "VAE encode ms @1024² (1024x1024 RGBA -> 64x64x64 latent), 1 GPU",
                           "value": rec["ms"], "unit": "ms/encode", "n_gpus": 1, "steps": steps, "warmup": warmup,
                           "higher_is_better": False, "dtype": "bf16", "data": "synthetic",
                           "config": {"workload": "vae-encode-1024x1024", "weights": "bf16 synthetic", "seed": SEED},
                           "weights_gb": round(vae_w / 1e9, 3), "scratch_gb": round(vae_s / 1e9, 2)}, **rec)),
          flush=True)


def vae_encode_record(t, finite):
    return {"ms": round(t * 1e3, 2), "tflop": round(VAE_ENC_FLOP / 1e12, 3),
            "tflops": round(VAE_ENC_FLOP / t / 1e12, 1),
            "mfma_peak_frac": round(VAE_ENC_FLOP / t / 1e12 / PEAK_TFLOPS, 4), "latent_finite": finite}


def vision_flop(n, d=1152, f=4304, depth=27, out=4096):
    """Multiply-add FLOPs of one vision encode of N patches: the patch embedding, each block's
    four products and attention's two (n x n x d each), the four mergers' two products."""
    m = n // 4
    blocks = depth * (2 * n * d * (3 * d + d + 2 * f) + 4 * n * n * d)
    return 2 * n * d * 768 + blocks + 4 * 2 * m * (4 * d * 4 * d + 4 * d * out)


def vision_time(ctx, reps, warmup, hh=1024, ww=1024):
    """The tower on a seeded hh x ww RGBA picture already in HBM: (ms an encode, finite, weights GB,
    scratch GB)."""
    import exn_hip as X
    rng = np.random.default_rng(SEED)
    vis = X.load_vision(seed=SEED, ctx=ctx)
    px = X.DevBuf.of(ctx, np.clip(rng.normal(0, 0.5, (hh, ww, 4)), -1, 1).astype(np.float32))
    m = (hh // 32) * (ww // 32)
    out = X.DevBuf(ctx, (4, m, 4096), np.float32)
    run = lambda: X.call("exn_vision_encode_dev", vis.h, px.h, hh, ww, out.h, out.at(m * 4096 * 4))
    for i in range(warmup):
        run()
    ctx.sync()
    t0 = time.perf_counter()
    for i in range(reps):
        run()
    ctx.sync()
    t = (time.perf_counter() - t0) / reps
    finite = bool(np.isfinite(out.get()).all())
    w, sc = vis.memory()
    vis.destroy()
    return t, finite, w / 1e9, sc / 1e9


def vision_record(t, finite, w_gb, s_gb, n=4096):
    fl = vision_flop(n)
    return {"ms": round(t * 1e3, 2), "tflop": round(fl / 1e12, 3), "tflops": round(fl / t / 1e12, 1),
            "f32_mfma_peak_frac": round(fl / t / 1e12 / PEAK_F32_TFLOPS, 4), "patches": n, "out_rows": n // 4,
            "outputs_finite": finite, "weights_gb": round(w_gb, 3), "scratch_gb": round(s_gb, 2)}


def encoder_flop(n, layers=36):
    """Multiply-add FLOPs of encoder-states over N tokens: per token and layer the products (q, k,
    v: 4096 -> 6144; out; gate and up; down) and causal attention's two (each token over itself
    and the tokens before it)."""
    return layers * (n * 2 * 4096 * (6144 + 4096 + 2 * 12288 + 12288) + 4 * 4096 * n * (n + 1) // 2)


def encoder_time(ctx, n, reps, warmup, picture_rows=0):
    """The prompt encoder (36 blocks, synthetic Q8_0 weights) over N tokens already in HBM, the
    last PICTURE_ROWS .. of them a picture's (merged rows and three deepstack sets, the vision
    tower's shapes, after 40 text tokens): ms per call."""
    import exn_hip as X
    rng = np.random.default_rng(SEED + n)
    enc = X.load_encoder(seed=SEED, layers=36, vocab=8192, ctx=ctx)
    ids = X.DevBuf.of(ctx, rng.integers(0, 8192, n).astype(np.int32))
    if picture_rows:
        a0, g = 40, int(round(picture_rows ** 0.5))
        r, c = np.divmod(np.arange(picture_rows), g)
        pos = np.concatenate([np.repeat(np.arange(a0)[:, None], 3, 1),
                              np.stack([np.full(picture_rows, a0), a0 + r, a0 + c], 1),
                              np.repeat(a0 + g + np.arange(n - a0 - picture_rows)[:, None], 3, 1)])
    else:
        a0, pos = 0, None
    cs = X.DevBuf.of(ctx, X.enc_rope_table(n, pos))
    pic = X.DevBuf.of(ctx, rng.normal(0, 1, (4, max(picture_rows, 1), 4096)).astype(np.float32))
    out = X.DevBuf(ctx, (n, 4096), np.float32)
    run = lambda: X.call("exn_enc_states_dev", enc.h, ids.h, n, cs.h, a0, picture_rows, pic.h,
                         pic.at(picture_rows * 4096 * 4), out.h)
    for i in range(warmup):
        run()
    ctx.sync()
    t0 = time.perf_counter()
    for i in range(reps):
        run()
    ctx.sync()
    t = (time.perf_counter() - t0) / reps
    finite = bool(np.isfinite(out.get()).all())
    w, _ = enc.memory()
    enc.destroy()
    fl = encoder_flop(n)
    return {"tokens": n, "picture_rows": picture_rows, "ms": round(t * 1e3, 2), "tflop": round(fl / 1e12, 3),
            "tflops": round(fl / t / 1e12, 1), "mfma_peak_frac": round(fl / t / 1e12 / PEAK_TFLOPS, 4),
            "states_finite": finite, "weights_gb": round(w / 1e9, 2)}


def pictures(ctx, d, reps=2):
    """Whole pictures on the device, as the reference's README times them (1024 x 1024, 1536 x
    1024, an edit at 1024 x 1024): the prompt's states from the encoder (synthetic ids), the
    8-step loop from fresh noise (a fresh prefix key: the first step uncached), the VAE decode to
    RGBA; an edit adds the vision tower on the picture to edit, whose merged and deepstack rows
    the encoder takes in the prompt, and the VAE encoder's latent of the picture, which the DiT
    takes beside the text's 512 states (the Lisp host's per-channel normalisation of that latent
    left out).  Each part is timed between synchronisations; ms a picture, the mean of REPS after
    one untimed picture."""
    import exn_hip as X
    rng = np.random.default_rng(SEED + 77)
    enc = X.load_encoder(seed=SEED, layers=36, vocab=8192, ctx=ctx)
    vis = X.load_vision(seed=SEED, ctx=ctx)
    vae = X.upload_vae(seed=SEED, ctx=ctx)
    sg = np.array(X.TURBO_SIGMAS, np.float64)
    recs = {}
    for name, (hh, ww, edit, ref_s) in {"1024sq": (64, 64, False, 11.0), "1536x1024": (96, 64, False, 22.0),
                                        "edit_1024sq": (64, 64, True, 20.0)}.items():
        ptext, a0, m = 512 if edit else P, 40, 1024 if edit else 0
        n = ptext + m
        ids = X.DevBuf.of(ctx, rng.integers(0, 8192, n).astype(np.int32))
        if edit:
            r, c = np.divmod(np.arange(m), 32)
            pos = np.concatenate([np.repeat(np.arange(a0)[:, None], 3, 1),
                                  np.stack([np.full(m, a0), a0 + r, a0 + c], 1),
                                  np.repeat(a0 + 32 + np.arange(n - a0 - m)[:, None], 3, 1)])
            px = X.DevBuf.of(ctx, np.clip(rng.normal(0, 0.5, (16 * hh, 16 * ww, 4)), -1, 1).astype(np.float32))
            vrows = X.DevBuf(ctx, (4, m, 4096), np.float32)
            rl = X.DevBuf(ctx, (64, hh, ww), np.float32)
        else:
            pos = None
        cs = X.DevBuf.of(ctx, X.enc_rope_table(n, pos))
        states = X.DevBuf(ctx, (n, 4096), np.float32)
        context = X.DevBuf(ctx, (ptext, 4096), np.float32) if edit else states
        noise = rng.normal(0, 1, (64, hh, ww)).astype(np.float32)
        z = X.DevBuf(ctx, (64, hh, ww), np.float32)
        pic = X.DevBuf(ctx, (16 * hh, 16 * ww, 4), np.float32)

        def picture():
            z.upload(noise)
            ctx.sync()
            t = [time.perf_counter()]
            if edit:
                X.call("exn_vision_encode_dev", vis.h, px.h, 16 * hh, 16 * ww, vrows.h, vrows.at(m * 4096 * 4))
                ctx.sync()
                t.append(time.perf_counter())
                X.call("exn_vae_encode_dev", vae.h, px.h, 16 * hh, 16 * ww, rl.h)
                ctx.sync()
                t.append(time.perf_counter())
                X.call("exn_enc_states_dev", enc.h, ids.h, n, cs.h, a0, m, vrows.h, vrows.at(m * 4096 * 4), states.h)
                # the text's states: the picture's rows left out
                X.call("exn_copy", ctx.h, context.h, states.h, a0 * 4096 * 4)
                X.call("exn_copy", ctx.h, context.at(a0 * 4096 * 4), states.at((a0 + m) * 4096 * 4),
                       (n - a0 - m) * 4096 * 4)
                refargs = (a0, rl.h, hh, ww)
            else:
                X.call("exn_enc_states_dev", enc.h, ids.h, n, cs.h, 0, 0, None, None, states.h)
                refargs = (0, None, 0, 0)
            ctx.sync()
            t.append(time.perf_counter())
            X.call("exn_dit_generate_dev", d.h, context.h, ptext, z.h, hh, ww, X.ptr(sg), len(sg), *refargs)
            ctx.sync()
            t.append(time.perf_counter())
            X.call("exn_vae_decode_dev", vae.h, z.h, hh, ww, pic.h)
            ctx.sync()
            t.append(time.perf_counter())
            return np.diff(t)

        picture()
        parts = np.mean([picture() for _ in range(reps)], axis=0) * 1e3
        names = (["vision_ms", "vae_encode_ms"] if edit else []) + ["encoder_ms", "dit_8_steps_ms", "vae_ms"]
        recs[name] = {"ms": round(float(parts.sum()), 1), **{k: round(float(v), 1) for k, v in zip(names, parts)},
                      "picture_h_x_w": "%d x %d" % (16 * hh, 16 * ww), "prompt_tokens": n, "text_rows": ptext,
                      "picture_finite": bool(np.isfinite(pic.get()).all()), "ref_rtx3090_s": ref_s}
        for b in [ids, cs, states, z, pic] + ([context, px, vrows, rl] if edit else []):
            b.free()
    enc.destroy()
    vis.destroy()
    vae.destroy()
    return recs


def vision_only(steps, warmup):
    """The vision tower alone: a seeded 1024 x 1024 RGBA picture in HBM -> merged + deepstack rows."""
    import exn_hip as X
    ctx = X.Context(0)
    t, finite, w_gb, s_gb = vision_time(ctx, steps, warmup)
    ctx.close()
    rec = vision_record(t, finite, w_gb, s_gb)
    print(json.dumps(dict({"metric": "vision encode ms @1024² (4096 patches, 27 blocks + 4 mergers), 1 GPU",
                           "value": rec["ms"], "unit": "ms/encode", "n_gpus": 1, "steps": steps, "warmup": warmup,
                           "higher_is_better": False, "dtype": "f32", "data": "synthetic",
                           "config": {"workload": "vision-encode-1024x1024", "weights": "fp16-valued synthetic, fp32",
                                      "seed": SEED}}, **rec)), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--vae-only", action="store_true", help="time the VAE decoder alone")
    ap.add_argument("--vae-encode-only", action="store_true", help="time the VAE encoder alone")
    ap.add_argument("--vision-only", action="store_true", help="time the vision tower alone")
    ap.add_argument("--encoder-only", action="store_true", help="time the prompt encoder alone")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="copy MIB MiB device to device after the set-up (the traffic counters' calibration)")
    ap.add_argument("--traffic-from", nargs=2, metavar=("FETCH_DB", "WRITE_DB"),
                    help="turn two rocprofv3 --pmc databases of a --copy-probe run into " + TRAFFIC_FILE +
                         " (with --q8-only: of the Q8_0 product, into " + TRAFFIC_FILE_Q8 + ")")
    ap.add_argument("--q8-only", action="store_true",
                    help="time only the cached step from Q8_0 weights (no resident bf16 copies, no VAE)")
    ap.add_argument("--uncached-only", action="store_true",
                    help="time the uncached step alone (the prompt rows through every block)")
    ap.add_argument("--w8a8-only", action="store_true",
                    help="time only the cached step in the reference's int8 mode (exn_dit_w8a8)")
    ap.add_argument("--bf16-only", action="store_true",
                    help="time only the cached step from the resident bf16 expansion (no other workloads, no VAE)")
    ap.add_argument("--power", type=float, default=0, metavar="SECONDS",
                    help="loop the cached step for SECONDS while sampling amd-smi's power and clocks "
                         "(with --q8-only: from Q8_0 weights)")
    ap.add_argument("--pmc-summary", nargs="+", metavar="DB",
                    help="print per-kernel clock and MFMA busy from rocprofv3 --pmc databases")
    a = ap.parse_args()
    if a.traffic_from:
        traffic_from(*a.traffic_from, q8=a.q8_only, bf16_only=a.bf16_only)
        return
    if a.pmc_summary:
        pmc_summary(a.pmc_summary)
        return
    if a.gpus != 1:
        print("bench.py: the step runs on one GPU; --gpus %d is not supported (a split of the image rows "
              "across GPUs is designed, not built)" % a.gpus, file=sys.stderr)
        sys.exit(2)
    if a.vision_only:
        vision_only(a.steps, a.warmup)
        return
    if a.encoder_only:
        import exn_hip as X
        ctx = X.Context(0)
        rec = {"prompt_256": encoder_time(ctx, 256, a.steps, a.warmup),
               "edit_1024sq": encoder_time(ctx, 1100, a.steps, a.warmup, 1024)}
        ctx.close()
        print(json.dumps({"metric": "prompt encoder ms (36 blocks of Qwen3-VL-8B's text model), 1 GPU",
                          "value": rec["prompt_256"]["ms"], "unit": "ms/prompt", "n_gpus": 1, "steps": a.steps,
                          "warmup": a.warmup, "higher_is_better": False, "dtype": "bf16", "data": "synthetic",
                          "config": {"workload": "encoder-states-256-tokens",
                                     "weights": "Q8_0 synthetic, the key/value heads once (q | k | v: 6144 rows); "
                                                "products of at most 256 rows stream the Q8_0 codes (the few-row "
                                                "kernel), longer ones the resident bf16 expansion "
                                                "(exn_enc_resident, the default; made by the first prompt "
                                                "of more than 256 tokens)",
                                     "seed": SEED}, "records": rec}), flush=True)
        return
    if a.vae_encode_only:
        vae_encode_only(a.steps, a.warmup)
        return
    if a.vae_only:
        vae_only(a.steps, a.warmup)
        return

    import exn_hip as X
    ctx = X.Context(0)
    d = X.Dit(ctx, LAYERS)
    ctx.sync()
    t0 = time.perf_counter()
    d.synth(SEED)   # synchronous: returns once the weights are made
    d.check()
    t1 = time.perf_counter()
    d.resident(not a.q8_only)   # synchronous too
    t2 = time.perf_counter()
    w_bytes, _ = d.memory()
    print("bench: synthetic 7B Q8_0 DiT made on the device in %.1f ms%s (%.1f GB of weights)"
          % ((t1 - t0) * 1e3, "" if a.q8_only else ", block matrices expanded to resident bf16 in %.1f ms"
             % ((t2 - t1) * 1e3), w_bytes / 1e9), file=sys.stderr, flush=True)
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

    if a.power:
        for i in range(1 + a.warmup):
            step(i, key)
        ctx.sync()
        power_run(a.power, step, ctx, z, latent, "Q8_0" if a.q8_only else "resident bf16 expansion")
        d.destroy()
        ctx.close()
        return
    if a.uncached_only:   # the uncached step alone: the prompt rows through every block too
        for i in range(1 + a.warmup):
            step(i, 0)
        ctx.sync()
        t0 = time.perf_counter()
        for i in range(a.steps):
            step(1 + i, 0)
        ctx.sync()
        t = (time.perf_counter() - t0) / a.steps
        tot = step_flops(False)[2]
        print(json.dumps({"metric": "DiT Euler step ms @1024², uncached (the 256 prompt rows through every block)",
                          "value": round(t * 1e3, 3), "unit": "ms/step", "steps": a.steps, "warmup": a.warmup,
                          "tflops": round(tot / t / 1e12, 1), "mfma_peak_frac": round(tot / t / 1e12 / PEAK_TFLOPS, 4),
                          "weights": "resident bf16 expansion; products of at most 256 rows from the Q8_0 codes"}),
              flush=True)
        d.destroy()
        ctx.close()
        return
    if a.w8a8_only:
        d.w8a8(True)
    if a.q8_only or a.bf16_only or a.w8a8_only:   # the cached step alone, for the profiles of one path
        for i in range(1 + a.warmup):
            step(i, key)
        ctx.sync()
        t0 = time.perf_counter()
        for i in range(a.steps):
            step(1 + i, key)
        ctx.sync()
        t = (time.perf_counter() - t0) / a.steps
        tot = step_flops(True)[2]
        what = ("Q8_0 weights (dequantised in the products)" if a.q8_only else
                "the reference's int8 products (exn_dit_w8a8)" if a.w8a8_only else "the resident bf16 expansion")
        print(json.dumps({"metric": "DiT Euler step ms @1024² from " + what,
                          "value": round(t * 1e3, 3), "unit": "ms/step", "steps": a.steps, "warmup": a.warmup,
                          "tflops": round(tot / t / 1e12, 1), "mfma_peak_frac": round(tot / t / 1e12 / PEAK_TFLOPS, 4),
                          "weights_gb": round(w_bytes / 1e9, 2)}), flush=True)
        d.destroy()
        ctx.close()
        return

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
    # the encoder (an edit's picture to its latent) on that picture
    t_venc, venc_ok = vae_encode_time(ctx, vae, pic, VAE_REPS, 1)
    vae_w, vae_s = vae.memory()
    vae.destroy()

    # the vision tower (editing's picture, seen by the prompt encoder) on a 1024 x 1024 picture,
    # and the prompt encoder on a 256-token prompt and on an edit prompt holding that picture's rows
    vis = vision_record(*vision_time(ctx, 3, 1))
    enc = {"prompt_256": encoder_time(ctx, 256, 3, 1), "edit_1024sq": encoder_time(ctx, 1100, 3, 1, 1024)}

    # the 1536 x 1024 and edit workloads on the same weights: cached and uncached steps
    def workload_times(hh, ww, ptext, ref, reps=3):
        r2 = np.random.default_rng(hh * ww + ptext)
        cx = X.DevBuf.of(ctx, r2.normal(0, 1, (ptext, 4096)).astype(np.float32))
        zc = X.DevBuf.of(ctx, r2.normal(0, 1, (64, hh, ww)).astype(np.float32))
        vc = X.DevBuf(ctx, (64, hh, ww), np.float32)
        if ref:
            ra, rh, rw = ref
            rl = X.DevBuf.of(ctx, r2.normal(0, 1, (64, rh, rw)).astype(np.float32))
            refargs = (ra, rl.h, rh, rw)
        else:
            refargs = (0, None, 0, 0)

        def vel(k, s):
            X.call("exn_dit_velocity_dev", d.h, cx.h, ptext, zc.h, hh, ww, s, k, *refargs, vc.h)

        vel(900, sig[0])              # the shape's workspace and K/V arrays allocated
        ctx.sync()
        t0 = time.perf_counter()
        for r in range(reps):         # uncached: a fresh key each call
            vel(901 + r, sig[0])
        ctx.sync()
        t_unc = (time.perf_counter() - t0) / reps
        vel(950, sig[0])              # the prompt's K/V kept under 950
        ctx.sync()
        t0 = time.perf_counter()
        for r in range(reps):
            vel(950, sig[1 + r % 7])
        ctx.sync()
        t_c = (time.perf_counter() - t0) / reps
        ok = bool(np.isfinite(vc.get()).all())
        nref = ref[1] * ref[2] if ref else 0
        fa = ref[0] if ref else 0
        fc = step_flops(True, hh * ww, ptext, nref, fa)[2]
        fu = step_flops(False, hh * ww, ptext, nref, fa)[2]
        return {"image_rows": hh * ww, "text_rows": ptext, "reference_rows": nref, "keys": ptext + nref + hh * ww,
                "cached_ms": round(t_c * 1e3, 2), "cached_tflop": round(fc / 1e12, 2),
                "cached_tflops": round(fc / t_c / 1e12, 1),
                "uncached_ms": round(t_unc * 1e3, 2), "uncached_tflop": round(fu / 1e12, 2),
                "uncached_tflops": round(fu / t_unc / 1e12, 1), "velocity_finite": ok}

    workloads = {"cfg3_1536x1024": workload_times(96, 64, 256, None),
                 "cfg4_edit_1024sq": workload_times(64, 64, 512, (8, 64, 64))}

    # whole pictures: prompt encoder, the 8-step loop and the VAE decode (an edit: the vision tower too)
    pics = pictures(ctx, d)

    # the same cached 1024^2 step with the block matrices multiplied from Q8_0: the codes
    # dequantised inside the products' pipeline, the resident bf16 copies dropped (the change of
    # product path drops the kept K/V too, so the first step recomputes them)
    d.resident(False)
    q8_w_bytes, _ = d.memory()
    for i in range(1 + a.warmup):
        step(1 + i, key)
    ctx.sync()
    d.profile(True, classes=["gate_up"], every=4)
    t0 = time.perf_counter()
    for i in range(a.steps):
        step(1 + i, key)
    ctx.sync()
    t_q8 = (time.perf_counter() - t0) / a.steps
    d.profile(False)
    q8_gu = d.profile_read()["gate_up"]
    d.profile(True, every=1)
    for i in range(BREAKDOWN):
        step(1 + i, key)
    ctx.sync()
    d.profile(False)
    q8prof = d.profile_read()

    # the reference's default *int8* products (exn_dit_w8a8), on the same Q8_0 weights: the
    # activations quantised to Q8_0 by blocks of 32 and multiplied on the int8 MFMA (the mode's
    # change drops the kept K/V, so the first step recomputes them)
    d.w8a8(True)
    for i in range(2):
        step(1 + i, key)
    ctx.sync()
    n8 = max(2, a.steps // 2)
    t0 = time.perf_counter()
    for i in range(n8):
        step(1 + i, key)
    ctx.sync()
    t_i8 = (time.perf_counter() - t0) / n8
    d.profile(True, every=1)
    step(1, key)
    ctx.sync()
    d.profile(False)
    i8prof = d.profile_read()
    d.w8a8(False)

    gemm_f, att_f, tot_f = step_flops(True)
    tflops = tot_f / (ms * 1e-3) / 1e12
    gu_ms, gu_n, gu_f, gu_b = gu_timed
    gu_avg = gu_ms / max(gu_n, 1)
    achieved = (gu_f / max(gu_n, 1)) / (gu_avg * 1e-3) / 1e12 if gu_n else None
    traffic = None
    if os.path.exists(TRAFFIC_FILE):
        traffic = json.load(open(TRAFFIC_FILE)).get("bytes_per_launch")
    def breakdown(pr, steps=BREAKDOWN):
        return {c: {"ms_per_step": round(pr[c][0] / steps, 3), "launches_per_step": pr[c][1] // steps,
                    **({"tflops": round(pr[c][2] / (pr[c][0] * 1e-3) / 1e12, 1)} if pr[c][2] else {}),
                    **({"gbs": round(pr[c][3] / (pr[c][0] * 1e-3) / 1e9, 1)} if pr[c][3] and not pr[c][2] else {})}
                for c in X.Dit.PROFILE_CLASSES if pr[c][1]}

    def gemm_rate(pr):
        g_ms = sum(pr[c][0] for c in ("qkv", "out", "gate_up", "down"))
        g_f = sum(pr[c][2] for c in ("qkv", "out", "gate_up", "down"))
        return g_f / (g_ms * 1e-3) / 1e12 if g_ms else None

    kernels = breakdown(prof)
    gemm_tf = gemm_rate(prof)
    q8_gu_avg = q8_gu[0] / max(q8_gu[1], 1)
    q8_gu_tf = (q8_gu[2] / max(q8_gu[1], 1)) / (q8_gu_avg * 1e-3) / 1e12 if q8_gu[1] else None
    q8_gemm_tf = gemm_rate(q8prof)
    q8 = {"ms_per_step": round(t_q8 * 1e3, 3), "tflops": round(tot_f / t_q8 / 1e12, 1),
          "mfma_peak_frac": round(tot_f / t_q8 / 1e12 / PEAK_TFLOPS, 4),
          "vs_resident_bf16": round(t_q8 * 1e3 / ms, 3),
          "weights_gb": round(q8_w_bytes / 1e9, 2),
          "gemm_tflops": round(q8_gemm_tf, 1) if q8_gemm_tf else None,
          "gemm_peak_frac": round(q8_gemm_tf / PEAK_TFLOPS, 4) if q8_gemm_tf else None,
          "gate_up": {"kernel": "gemm gate_up + SwiGLU, 4096 x 24576 x 4096, Q8_0 weights dequantised in the pipeline "
                                "(512 x 128 tiles)",
                      "achieved": round(q8_gu_tf, 1) if q8_gu_tf else None, "unit": "TFLOP/s",
                      "frac": round(q8_gu_tf / PEAK_TFLOPS, 4) if q8_gu_tf else None,
                      "avg_launch_ms": round(q8_gu_avg, 4), "launches_timed": q8_gu[1]},
          "kernels": breakdown(q8prof)}
    i8_gemm_tf = gemm_rate(i8prof)
    w8a8 = {"ms_per_step": round(t_i8 * 1e3, 3), "tflops": round(tot_f / t_i8 / 1e12, 1),
            "vs_resident_bf16": round(t_i8 * 1e3 / ms, 3),
            "gemm_tops": round(i8_gemm_tf, 1) if i8_gemm_tf else None,
            "note": "the reference's default *int8* products: activations quantised to Q8_0 by blocks of 32, "
                    "int8 MFMA with an fp32 rescale a block (VALU-bound on gfx950)",
            "kernels": breakdown(i8prof, 1)}
    out = {
        "metric": METRIC, "value": round(ms, 3), "unit": "ms/step", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(ms, 3), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "dit-euler-step-1024x1024", "image_rows": H * W, "text_rows": P, "blocks": LAYERS,
                   "weights": "Q8_0 synthetic (7.0B block + 0.14B edge parameters); the block products stream "
                              "each matrix's resident bf16 expansion bf16(fp32(d) q), 14 GB beside the 7.4 GB "
                              "of Q8_0 (the q8_0 key: the same step from Q8_0 alone)",
                   "step": "cached: image rows over kept prompt K/V, + Euler update", "seed": SEED},
        "tflops": round(tflops, 1), "mfma_peak_frac": round(tflops / PEAK_TFLOPS, 4),
        "step_tflop": round(tot_f / 1e12, 3),
        "gemm_tflops": round(gemm_tf, 1) if gemm_tf else None,
        "gemm_peak_frac": round(gemm_tf / PEAK_TFLOPS, 4) if gemm_tf else None,
        "first_call_ms": round(t_first * 1e3, 2), "uncached_step_ms": round(t_uncached * 1e3, 2),
        "euler_8_steps_ms": round(t_8 * 1e3, 1),
        "host_boundary_velocity_ms": round(t_host, 3),
        "final_latent_finite": finite, "ref_rtx3090_ms_per_step": 1187.5,
        "kernels": kernels,
        "q8_0": q8,
        "w8a8": w8a8,
        "workloads": workloads,
        "pictures": pics,
        "vae_decode_1024sq": {"ms": round(t_vae * 1e3, 2), "tflop": round(VAE_FLOP / 1e12, 2),
                              "tflops": round(VAE_FLOP / t_vae / 1e12, 1),
                              "mfma_peak_frac": round(VAE_FLOP / t_vae / 1e12 / PEAK_TFLOPS, 4),
                              "picture_finite": bool(np.isfinite(px).all()),
                              "weights_gb": round(vae_w / 1e9, 3), "scratch_gb": round(vae_s / 1e9, 2),
                              "ref_rtx3090_ms": 1500.0},
        "vae_encode_1024sq": vae_encode_record(t_venc, venc_ok),
        "vision_encode_1024sq": vis,
        "prompt_encoder": enc,
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
