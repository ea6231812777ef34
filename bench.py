#!/usr/bin/env python3
"""Throughput of the Big-LaMa FP32 generator forward on one MI355X.

Workload: one 512x512 whole-image pass, batch 1,
seeded random-init weights of the real architecture (989 tensors), a seeded
blurred-noise image with a ~25% brush-stroke mask.  A "step" is one forward
pass; the input tensor is resident in HBM before the timed region starts.

Prints one JSON line: passes/s, the roofline of the dominant kernel (the FFC
3x3 convolutions as Winograd F(4,3) along x, F(2x4, 3x3) on the bottleneck
planes of 1024x1024 inputs and up: the FLOPs of that algorithm's MFMA
products per launch / mean launch time on the device clock, against the
157.3 TFLOP/s FP32 MFMA peak; the direct-convolution equivalent rate beside
it), the host enqueue time of one pass, the wall time of the lama-inpaint
command on the reference's published case (2048x2048 image, 300x300 hole,
whole image and --tile) beside the reference's own figures, and the CPU
baseline (the C restatement of the reference CPU engine, timed on this host's
cores: median of three passes at 512x512 and at 256x256).
"""
import argparse
import json
import shutil
import subprocess
import os
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_FP32_MFMA = 157.3  # TFLOP/s, MI355X dense FP32 matrix
PEAK_HBM = 8000.0  # GB/s
# The reference's only published timings of this path (README.md:78-79): one
# run of its binary on a 2048x2048 image with a 300x300 hole, whole image and
# --tile (one 600x600 window), on a GTX 1080.
REF_CLI_S = {"whole": 4.58, "tile": 0.67}


def cli_wall_times(H, wpath, tmp, reps=3):
    """Wall time of this build's lama-inpaint on the reference's published case:
    a 2048x2048 image with a seeded 300x300 hole, whole image and --tile, each
    a fresh process (start-up, weight file read, packing and upload, PNG
    decode and encode included), `reps` runs each.  Beside them, configs[4]'s
    other case, for which the reference publishes no time: --sections on the
    same image with a seeded 1024x1024 hole (16 passes of 512x512)."""
    cli = os.path.join(ROOT, "lama-inpaint-rs_amd", "bin", "lama-inpaint")
    img = H.synth_image(2048, 2048, 1)
    mask, _ = H.synth_mask_rect(2048, 2048, 300, 300, 2)
    ip, mp = os.path.join(tmp, "in2048.png"), os.path.join(tmp, "mask2048.png")
    H.png_write_rgb(ip, img)
    H.png_write_rgb(mp, np.repeat(mask[..., None], 3, -1))
    big, _ = H.synth_mask_rect(2048, 2048, 1024, 1024, 2)
    mpb = os.path.join(tmp, "mask2048_1024.png")
    H.png_write_rgb(mpb, np.repeat(big[..., None], 3, -1))
    runs = {}
    for mode, m, extra in (("whole", mp, []), ("tile", mp, ["--tile"]), ("sections", mpb, ["--sections"])):
        op = os.path.join(tmp, f"out2048_{mode}.png")
        ts = []
        for _ in range(reps):
            t = time.perf_counter()
            p = subprocess.run([cli, "--image", ip, "--mask", m, "--output", op, "--weights", wpath, "--gpu",
                                *extra], capture_output=True, timeout=300)
            ts.append(time.perf_counter() - t)
            if p.returncode != 0:
                raise RuntimeError(f"lama-inpaint {mode} failed ({p.returncode}): "
                                   + p.stderr.decode(errors="replace")[-400:])
        runs[mode] = ts
    return {"whole_s": round(float(np.median(runs["whole"])), 3),
            "tile_s": round(float(np.median(runs["tile"])), 3),
            "sections_1024_hole_s": round(float(np.median(runs["sections"])), 3),
            "runs_s": {m: [round(v, 3) for v in ts] for m, ts in runs.items()},
            "reference_gtx1080_s": REF_CLI_S,
            "speedup_vs_reference": {m: round(REF_CLI_S[m] / float(np.median(runs[m])), 2) for m in REF_CLI_S},
            "case": ("lama-inpaint-rs_amd/bin/lama-inpaint --gpu [--tile] on a 2048x2048 synthetic image with a "
                     "seeded 300x300 hole (README.md:78-79's case), synthetic weights; wall time of each "
                     f"process, median of {reps}; the reference's figures are its README's, on a GTX 1080; "
                     "sections_1024_hole_s: --sections on the same image with a seeded 1024x1024 hole "
                     "(BASELINE configs[4], 16 passes of 512x512; no published reference time)")}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--size", type=int, default=512)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-cli", action="store_true",
                    help="skip the command-line wall times (2048x2048 image, 300x300 hole, whole and --tile)")
    ap.add_argument("--cpu-size", type=int, default=0, help="CPU sample size (default: the workload size)")
    ap.add_argument("--traffic", type=str, default=os.path.join(ROOT, "profiles", "traffic_conv3x3_512.json"),
                    help="JSON with the measured HBM bytes per launch of the dominant kernel")
    ap.add_argument("--sample-every", type=int, default=16,
                    help="time the dominant kernel's launches (HIP events in the dispatch packets) on every "
                         "N-th timed pass")
    ap.add_argument("--copy-probe", type=int, default=0,
                    help="MiB of one untimed device-to-device copy made before the warmup: the known-size "
                         "kernel that scales the FETCH_SIZE / WRITE_SIZE counters")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this backend runs one forward on one GPU; multi-GPU runs are not part of this build "
              "(a batch-1 pass does not shard across GPUs)", file=sys.stderr)
        sys.exit(2)

    import __graft_entry__

    pkg = __graft_entry__.load_package()
    H = pkg.host_api
    E = pkg.hip_engine
    S = args.size

    tmp = tempfile.mkdtemp(prefix="lama_bench_")
    wpath = os.path.join(tmp, "big-lama-synth.safetensors")
    H.synth_weights(wpath, 0)
    store = H.Store(wpath)
    eng = E.Engine()
    eng.load_weights(store)

    img = H.synth_image(S, S, 1)
    mask, coverage = H.synth_mask_strokes(S, S, 0.25, 2)
    x = H.build_input(img, mask)
    d_in = eng.malloc(x.nbytes)
    d_out = eng.malloc(3 * S * S * 4)
    eng.upload(d_in, x)

    if args.copy_probe:
        nb = args.copy_probe << 20
        a, b = eng.malloc(nb), eng.malloc(nb)
        eng.copy_d2d(b, a, nb)
        eng.synchronize()
        eng.free(a)
        eng.free(b)

    for _ in range(args.warmup):
        eng.forward_device(d_in, S, S, d_out)
    eng.synchronize()

    # The dominant kernel is timed with HIP events on its own stream during the
    # timed region, on every --sample-every-th pass (the events ride in the
    # dispatch packets; sampling keeps their cost out of `value`).
    # both launches of each FFC: A = l2l + l2g (family conv3x3) and B = g2l
    # (family conv3x3g2l), one kernel
    dom_fams = ["conv3x3", "conv3x3g2l"]
    # the FFC 3x3 convolutions run as Winograd F(4,3) along x, or F(2x4, 3x3)
    # on bottleneck planes of 128 x 128 and up (LAMA_FFC_WINO=2: F(2,3); 0:
    # the direct implicit GEMM; 4 / 42 force one Winograd form everywhere).
    # The engine counts each launch's direct-convolution FLOPs, 2 Cin Cout 9 H
    # W; the algorithm's own MFMA products are the fraction `issued` of that:
    # F(4,3) multiplies 6 transformed positions x 3 kernel rows per 4 output
    # pixels (18 of the direct 36 products, 1/2), F(2,3) 4 x 3 per 2 (12 of
    # 18, 2/3), F(2x4, 3x3) 4 x 6 positions per 2 x 4 pixels (24 of 72, 1/3).
    # The plan's own kernel for the FFC GEMMs at this size names the
    # algorithm (and the F(4,3) block shape, chosen per plane: 2 x 64, 4 x 32
    # or 8 x 16 output pixels).
    dom_kernel = eng.kernel_name(S, S, "conv3x3")
    wino = {"lama_conv3x3": 0, "lama_conv3x3w": 2, "lama_conv3x3w42": 42}.get(dom_kernel, 4)
    issued = {0: 1.0, 2: 2.0 / 3.0, 4: 0.5, 42: 1.0 / 3.0}[wino]
    block = {"lama_conv3x3": "64 px", "lama_conv3x3w": "2 rows x 64 px", "lama_conv3x3w4": "2 rows x 64 px",
             "lama_conv3x3w4n": "4 rows x 32 px", "lama_conv3x3w4q": "8 rows x 16 px",
             "lama_conv3x3w42": "4 rows x 64 px"}[dom_kernel]
    geometry = "workgroups of 64 channels x " + block
    method = {0: "direct implicit GEMM", 2: "Winograd F(2,3) along x", 4: "Winograd F(4,3) along x",
              42: "Winograd F(2x4, 3x3)"}[wino]
    eng.profile_reset()
    eng.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        eng.profile(dom_fams if i % args.sample_every == 0 else ())
        eng.forward_device(d_in, S, S, d_out)
    eng.synchronize()
    elapsed = time.perf_counter() - t0
    prof = eng.profile_read()
    eng.profile(())

    # per-family device times in one extra (untimed) profiled pass set
    eng.profile(E.FAMILIES)
    eng.profile_reset()
    for _ in range(3):
        eng.forward_device(d_in, S, S, d_out)
    eng.synchronize()
    fam = eng.profile_read()
    eng.profile(())

    # host enqueue time of one pass: the launch loop alone (forward_device
    # returns once every launch is queued), on an idle device so that no
    # queue back-pressure is counted; the pass's device time beside it
    enq, walls = [], []
    for _ in range(max(5, min(20, args.steps))):
        eng.synchronize()
        t = time.perf_counter()
        eng.forward_device(d_in, S, S, d_out)
        t1 = time.perf_counter()
        eng.synchronize()
        enq.append(t1 - t)
        walls.append(time.perf_counter() - t)
    enqueue_ms = float(np.median(enq)) * 1e3
    isolated_ms = float(np.median(walls)) * 1e3

    out = np.empty((3, S, S), np.float32)
    eng.download(out, d_out)
    assert np.isfinite(out).all()

    # PCIe-inclusive rates: the CLI's path, lama_hip_inpaint (u8 image and
    # mask in, u8 composite out; build_input and composite on the device),
    # and lama_hip_forward (f32 [4][h][w] in, f32 [3][h][w] out)
    n_io = max(3, min(10, args.steps))
    eng.inpaint(img, mask)
    t = time.perf_counter()
    for _ in range(n_io):
        u8 = eng.inpaint(img, mask)
    host_io = n_io / (time.perf_counter() - t)
    assert np.array_equal(u8, H.composite(img, mask, out, 0, 0))
    t = time.perf_counter()
    for _ in range(n_io):
        host_out = eng.forward(x)
    host_f32_io = n_io / (time.perf_counter() - t)
    assert np.array_equal(host_out, out)

    # the SpectralTransform alone, FFCs 0..17 (distinct
    # weights) on 384 x (S/8)^2 N(0,1) inputs resident in HBM, back to back
    # on one stream
    h8 = S // 8
    xs = np.random.default_rng(1000).standard_normal((384, h8, h8)).astype(np.float32)
    d_xs, d_ys = eng.malloc(xs.nbytes), eng.malloc(xs.nbytes)
    eng.upload(d_xs, xs)
    for k in range(18):
        eng.spectral_device(k, d_xs, h8, h8, d_ys)
    eng.synchronize()
    reps = 5
    t = time.perf_counter()
    for _ in range(reps):
        for k in range(18):
            eng.spectral_device(k, d_xs, h8, h8, d_ys)
    eng.synchronize()
    spec_us = (time.perf_counter() - t) * 1e6 / (reps * 18)
    eng.free(d_xs)
    eng.free(d_ys)

    ms = elapsed * 1e3 / args.steps
    # the dominant kernel's launches, A and B, each timed by its kernel-clock
    # window (first workgroup start to last workgroup end: the interval a
    # kernel trace reports for the dispatch).  The HIP event interval is
    # reported beside it for A (which waits on no other stream): it also holds
    # the launch's dispatch latency.  B's event interval would start at its
    # cross-stream wait.
    dA, dB = prof["conv3x3"], prof["conv3x3g2l"]
    n_clock = dA.get("clock_launches", 0) + dB.get("clock_launches", 0)
    n_dom = dA["launches"] + dB["launches"]
    flops_launch = (dA["flops"] + dB["flops"]) / max(1, n_dom)
    launch_ms_events_a = dA["ms"] / max(1, dA["launches"])
    if n_clock == n_dom and n_clock > 0:
        launch_ms = (dA["clock_ms"] + dB["clock_ms"]) / n_clock
        clock_a = dA["clock_ms"] / dA["clock_launches"]
        clock_b = dB["clock_ms"] / dB["clock_launches"]
    else:  # no stamps read: A's events alone
        launch_ms = launch_ms_events_a
        flops_launch = dA["flops"] / max(1, dA["launches"])
        clock_a = clock_b = None
    # the Winograd algorithm's FLOPs (its MFMA products) per launch, and the
    # direct-convolution count the same launch replaces
    exec_launch = flops_launch * issued
    achieved = exec_launch / (launch_ms * 1e-3) / 1e12
    achieved_direct = flops_launch / (launch_ms * 1e-3) / 1e12
    traffic = None
    if args.traffic and os.path.exists(args.traffic):
        with open(args.traffic) as fh:
            t = json.load(fh)
        # only a measurement of the same kernel and launch shapes applies
        if (t.get("kernel") == dom_kernel and t.get("size") == S
                and abs(t.get("flops_per_launch", 0) - flops_launch) <= 1e-6 * flops_launch):
            traffic = t["bytes_per_launch"]

    conv_fams = ["conv7x7", "conv3x3s2", "conv3x3", "conv3x3g2l", "conv1x1", "convt", "conv1x1res"]
    conv_flops = sum(fam[f]["flops"] for f in conv_fams) / 3
    # executed MFMA work: the Winograd FFC families at the fraction `issued`
    # of their direct-convolution FLOPs (1/2 for F(4,3), 2/3 for F(2,3), 1/3
    # for F(2x4, 3x3))
    wino_fams = ("conv3x3", "conv3x3g2l")
    conv_flops_exec = conv_flops - sum(fam[f]["flops"] for f in wino_fams) / 3 * (1.0 - issued)
    fft_ms = sum(fam[f]["ms"] for f in ("rfft2", "irfft2")) / 3
    fft_bytes = sum(fam[f]["bytes"] for f in ("rfft2", "irfft2")) / 3
    # event time per family; a launch issued after a cross-stream wait (every
    # conv3x3g2l, conv1x1res and finalize launch; the pass's first spectral
    # conv1x1 and first convt) is timed from the wait, so it includes it
    per_family = {f: {"ms_per_pass": round(v["ms"] / 3, 4), "launches_per_pass": v["launches"] // 3,
                      "tflops": round(v["flops"] / (v["ms"] * 1e9), 2) if v["ms"] > 0 else None,
                      "gbps": round(v["bytes"] / (v["ms"] * 1e6), 1) if v["ms"] > 0 else None,
                      "clock_ms_per_pass": round(v["clock_ms"] / 3, 4) if v.get("clock_launches") else None}
                  for f, v in fam.items()}

    cpu = None
    if not args.no_cpu:
        sys.path.insert(0, os.path.join(ROOT, "tests"))
        import oracle_api as O

        cs = args.cpu_size or S
        net = O.OracleNet(O.read_safetensors(wpath))

        def cpu_passes(n, reps=3):
            """Seconds of `reps` whole-image passes at n x n (weights preloaded)."""
            cimg = H.synth_image(n, n, 1)
            cmask, _ = H.synth_mask_strokes(n, n, 0.25, 2)
            cx = H.build_input(cimg, cmask)
            ts = []
            for _ in range(reps):
                t = time.perf_counter()
                net.forward(cx)
                ts.append(time.perf_counter() - t)
            return ts

        # the workload size, median of three; 256x256 (configs[0]'s shape) beside it
        cpu_ts = cpu_passes(cs)
        cpu_s = float(np.median(cpu_ts))
        cpu_ts256 = cpu_passes(256) if cs != 256 else cpu_ts
        scale = (cs / S) ** 2  # work scales with the pixel count
        cpu_model = "unknown"
        try:
            with open("/proc/cpuinfo") as fh:
                for ln in fh:
                    if ln.startswith("model name"):
                        cpu_model = ln.split(":", 1)[1].strip()
                        break
        except OSError:
            pass
        # lscpu's identification lines, where the box has the tool
        lscpu = {}
        try:
            out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
            for ln in out.splitlines():
                k, _, v = ln.partition(":")
                if k.strip() in ("Model name", "Vendor ID", "CPU family", "Model", "Stepping", "CPU(s)",
                                 "Thread(s) per core", "Core(s) per socket", "Socket(s)", "CPU max MHz",
                                 "L3 cache", "Hypervisor vendor", "Virtualization type"):
                    lscpu[k.strip()] = v.strip()
        except (OSError, subprocess.SubprocessError):
            pass
        cpu = {"value": round(scale / cpu_s, 5), "unit": "passes/s", "cores": O.lib().or_num_threads(),
               "cpu_model": cpu_model, "lscpu": lscpu, "kind": "port",
               "sample": f"median of three {cs}x{cs} whole-image passes of the C restatement of cpu.rs "
                         f"(-O3 -ffp-contract=off, OpenMP, weights preloaded): {cpu_s:.2f} s"
                         + ("" if cs == S else f", scaled by pixel count to {S}x{S}"),
               "pass_s": [round(v, 3) for v in cpu_ts],
               "passes_per_s_256": round(1.0 / float(np.median(cpu_ts256)), 4),
               "pass_s_256": [round(v, 3) for v in cpu_ts256]}

    line = {
        "metric": f"{S}x{S} inpaint passes/sec (FP32, batch 1)",
        "value": round(args.steps / elapsed, 3),
        "unit": "passes/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded random-init Big-LaMa weights, blurred-noise image, brush-stroke mask)",
        "config": {"workload": f"Big-LaMa generator whole-image pass {S}x{S}, batch 1"
                               + {512: " (BASELINE configs[3])", 2048: " (BASELINE configs[4])",
                                  256: " (BASELINE configs[0] shape)"}.get(S, ""),
                   "h": S, "w": S, "mask_coverage": round(coverage, 4), "launches_per_pass": eng.launch_count(S, S)},
        "roofline": {"bound": "mfma",
                     "kernel": (dom_kernel + f" (FFC 3x3 convolutions as {method}, {geometry}"
                                + "; timed: both launches of every FFC of the sampled passes, A = l2l + l2g "
                                  "and B = g2l, each from its first workgroup's start to its last workgroup's end "
                                  "on the device clock; they overlap each other and the spectral branch on three "
                                  "streams, so a duration includes the time the launch shares the CUs)"),
                     "achieved": round(achieved, 2), "peak": PEAK_FP32_MFMA, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_FP32_MFMA, 4), "traffic": traffic,
                     "flops_kind": (f"the {method} algorithm's MFMA products, {issued:.4g} of the direct "
                                    "convolution's 2 Cin Cout 9 H W"),
                     "flops_per_launch": exec_launch,
                     "direct_flops_per_launch": flops_launch,
                     "achieved_direct_equivalent": round(achieved_direct, 2),
                     "launch_ms": round(launch_ms, 5),
                     "launch_ms_source": ("kernel clock (s_memrealtime stamps of every workgroup)"
                                          if clock_a is not None else "HIP events (A launches)"),
                     "launches_timed": int(n_dom),
                     "launch_ms_a": round(clock_a, 5) if clock_a is not None else None,
                     "launch_ms_b": round(clock_b, 5) if clock_b is not None else None,
                     "launch_ms_a_events": round(launch_ms_events_a, 5)},
        # all conv families' direct-convolution FLOPs over the pass's wall
        # time, and the MFMA work actually executed (the Winograd families at
        # `issued`) over the same time
        "pass_conv_tflops": round(conv_flops / (ms * 1e9), 2),
        "pass_conv_frac_of_peak": round(conv_flops / (ms * 1e9) / PEAK_FP32_MFMA, 4),
        "pass_conv_flops_kind": "direct convolution (2 Cin Cout Kh Kw Hout Wout)",
        "pass_conv_executed_tflops": round(conv_flops_exec / (ms * 1e9), 2),
        "pass_conv_executed_frac_of_peak": round(conv_flops_exec / (ms * 1e9) / PEAK_FP32_MFMA, 4),
        "fft_gbps": round(fft_bytes / (fft_ms * 1e6), 1) if fft_ms > 0 else None,
        "fft_frac_of_hbm": round(fft_bytes / (fft_ms * 1e6) / PEAK_HBM, 4) if fft_ms > 0 else None,
        "host_io_passes_per_s": round(host_io, 3),
        "host_io_path": "lama_hip_inpaint: u8 image + mask in, u8 composite out (PCIe-inclusive)",
        "host_f32_io_passes_per_s": round(host_f32_io, 3),
        "host_enqueue_ms_per_pass": round(enqueue_ms, 4),
        "isolated_pass_ms": round(isolated_ms, 4),
        "host_enqueue_note": ("host time of forward_device (the launch loop alone, device idle at the call), "
                              "median; isolated_pass_ms: the same call through its synchronize"),
        "spectral_block_us": round(spec_us, 2),
        "spectral_block_workload": f"BASELINE configs[2]: SpectralTransform of FFCs 0..17 on 384x{h8}x{h8}, "
                                   "conv1 -> rfft2 -> FU conv -> irfft2 -> conv2, one stream",
        "per_family": per_family,
        "cpu_baseline": cpu,
    }
    eng.free(d_in)
    eng.free(d_out)
    eng.close()
    # the command line runs as the README times it: each process alone on the
    # device (this process's engine closed first)
    line["cli_2048"] = None if args.no_cli else cli_wall_times(H, wpath, tmp)
    line["cpu_baseline"] = line.pop("cpu_baseline")
    print(json.dumps(line), flush=True)
    shutil.rmtree(tmp, ignore_errors=True)


if __name__ == "__main__":
    main()
