"""Throughput of the MI355X swin2sr backend on the north-star workload.

python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--workload W]

Workload (BASELINE.json metric): Swin2SR classical x4, fp32, a 256x256 RGB
input upscaled to 1024x1024, whole image, one GPU. Weights are random-init by
the benchmark's rules (seed 3; there is no published checkpoint offline) and
the input is config 2's generator (8 random 2-D sinusoids + N(0, 4^2) noise,
clipped to u8) at 256x256, seed 3. A step is one whole-image forward
(s2s_forward_device: padding, 36 Swin blocks, 6 RSTB closes, the head, the
denormalise/crop) from an HBM-resident mean-adjusted input to an HBM-resident
output; the timed steps replay the HIP graph the library captures for a
repeated call.

One JSON line on stdout. `roofline` is for the kernel with the largest share
of device time per step, its launches timed with HIP events on the library's
own stream (a pair around every launch of K forwards launched kernel by
kernel, before the timed replays); `cpu_baseline` is
this repository's C restatement of the crate's CPU path (oracle/, OpenMP over
the host cores) on a bounded sample. The replayed output is checked bit for
bit against an eager forward of the same input; a mismatch fails the run.

Other workloads (--workload), each one JSON line of the same shape: rstb
(config 1, one RSTB on an unpadded 256x256x180 plane), lightweight-x2,
classical-x2 and realworld-x4 (configs 0, 2, 3, whole image, HBM-resident),
compressed-x4-tiled (config 4: 1024x1024 in 256-pixel tiles with 64 of
context through the crate's tile loop over the host-buffer entry).
"""
import argparse
import hashlib
import json
import os
import re
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

import __graft_entry__ as ge  # noqa: E402

METRIC = "output Mpix/s classical-x4 256²→1024² fp32 @1 GPU; % MFMA / HBM roofline"
MFMA_FP32_PEAK = 157.3e12   # MI355X dense fp32 matrix, FLOP/s (AMD spec)
HBM_PEAK = 8.0e12           # MI355X HBM3E, B/s (AMD spec)
VALU_FP32_PEAK = 78.6e12    # MI355X fp32 vector FMA (256 CUs x 4 SIMDs x 16 lanes x 2 x 2.4 GHz)
FLOP_PEAK = {"mfma": MFMA_FP32_PEAK, "valu": VALU_FP32_PEAK}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def kernel_work(arch, h, w, hp=None, wp=None):
    """Algorithmic work per launch of each named kernel: (bound, flops, bytes).
    FLOPs count 2 per multiply-add over the real (unpadded) GEMM extents on the
    padded plane; bytes are the minimum unique fp32 reads + writes. (hp, wp)
    default to the padded plane of an h x w image."""
    win, C, s, F = arch.window, arch.embed, arch.scale, arch.feat
    if hp is None:
        hp, wp = (h // win + 1) * win, (w // win + 1) * win
    P = hp * wp
    VT = 36 * ((hp + 3) // 4) * ((wp + 3) // 4)  # rows of the 36 Winograd GEMMs
    Hd = arch.mlp_ratio * C
    f = 4
    work = {
        "qkv": ("mfma", 2 * P * 3 * C * C, f * P * (C + 3 * C)),
        # 6 heads of 30: the qkv projection and the window attention as one
        # kernel (x in, the attention output out; q, k, v stay on the CU)
        "qkv_window_attention": ("mfma", 2 * P * 3 * C * C + 4 * P * win * win * C,
                                 f * (P * 2 * C + 3 * C * C)),
        "window_attention": ("mfma", 4 * P * win * win * C, f * P * (3 * C + C)),
        "proj_ln_res": ("mfma", 2 * P * C * C, f * P * 3 * C),
        "fc1_gelu": ("mfma", 2 * P * Hd * C, f * P * (C + Hd)),
        "fc2_ln_res": ("mfma", 2 * P * C * Hd, f * P * (Hd + 2 * C)),
        # the body's 3x3 convs (the stage close with the 1x1 folded in, and
        # conv_after_body) as Winograd F(4x4,3x3) over T = ceil(hp/4) ceil(wp/4)
        # tiles: the input transform (the plane in, 36 transform planes of T
        # tiles out), the 36 transform-position GEMMs (T x C x C multiply-adds
        # each: 72 T C^2 FLOPs, the direct conv's 18 P C^2 / 4 when 4 divides
        # the plane; M over V in place), then the output transform + bias +
        # residual (M and the residual in, the plane out)
        "conv3x3_stage_in": ("hbm", 0, f * (P * C + VT * C)),
        "conv3x3_stage": ("mfma", 2 * VT * C * C, f * (2 * VT * C + 36 * C * C)),
        "conv3x3_stage_out": ("hbm", 0, f * (VT * C + 2 * P * C)),
        "conv_after_body_in": ("hbm", 0, f * (P * C + VT * C)),
        "conv_after_body": ("mfma", 2 * VT * C * C, f * (2 * VT * C + 36 * C * C)),
        "conv_after_body_out": ("hbm", 0, f * (VT * C + 2 * P * C)),
        # conv_first and patch_embed (its 1x1 folded into conv_first) + LayerNorm
        # in one pass on fp32 MFMA: two K = 27 convs
        "embed": ("mfma", 2 * 2 * P * C * 27, f * P * (4 + 2 * C)),
        "layernorm": ("hbm", 10 * P * C, f * P * 2 * C),
        "pad_input": ("hbm", 0, f * (3 * h * w + 4 * P)),
        "conv_last_finish": ("hbm", 2 * (h * s) * (w * s) * 3 * 9 * F,
                             f * ((hp * s) * (wp * s) * F + 3 * h * s * w * s)),
        # the last octave and conv_last composed: 12 outputs from a 5x5xF
        # footprint per input pixel whose outputs survive the crop (VALU)
        "up_last": ("valu", 2 * (h * s // 2) * (w * s // 2) * 12 * 25 * F,
                    f * ((hp * s // 2) * (wp * s // 2) * F + 3 * h * s * w * s)),
        # the last two octaves and conv_last composed: a 5x5 conv GEMM to 48
        # outputs per pixel of the plane before them (scale 4), over the rows
        # whose outputs survive the crop (ceil(oh / 4) of them)
        "up2_last": ("mfma", 2 * min(hp * s // 4, -(-h * s // 4)) * (wp * s // 4) * 48 * 25 * F,
                     f * ((hp * s // 4) * (wp * s // 4) * F + 3 * h * s * w * s)),
    }
    shuffle = arch.upsampler in ("pixelshuffle", "pixelshuffle_aux")
    if shuffle and s == 4 and F == 64:
        # the x4 head's composed 5x5 conv as Winograd F(2x2,5x5) over the
        # T5 2x2 tiles of the pixels whose outputs survive the crop: the input
        # transform (the plane in, 36 planes of T5 x F out), 36 GEMMs of
        # T5 x 48 x F, the output transform (M in, the cropped image out)
        ho, wo = min(hp, -(-h * s // 4)), min(wp, -(-w * s // 4))
        T5 = 36 * ((ho + 1) // 2) * ((wo + 1) // 2)
        work["up2_last_in"] = ("hbm", 0, f * (ho * wo * F + T5 * F))
        work["up2_last"] = ("mfma", 2 * T5 * 48 * F, f * (T5 * (F + 48) + 36 * 48 * F))
        work["up2_last_out"] = ("hbm", 0, f * (T5 * 48 + 3 * h * s * w * s))
    if shuffle and s >= 4 and F == 64:
        # input row 0 and column 0 recomputed with the padding-aware variants:
        # 48 outputs of a 5x5xF footprint per border pixel (VALU)
        nb = -(-h * s // 4) + -(-w * s // 4) - 1
        work["up2_last_edge"] = ("valu", 2 * nb * 48 * 25 * F, f * (nb * 25 * F + 4 * 48 * 25 * F))
    if C in (60, 120, 180) and F % 4 == 0 and F <= 64:
        # conv_before_upsample (C -> F, LeakyReLU) as Winograd F(4x4,3x3): the
        # same input transform, 36 GEMMs of T x F x C, the output transform
        work["conv_before_upsample_in"] = ("hbm", 0, f * (P * C + VT * C))
        work["conv_before_upsample"] = ("mfma", 2 * VT * F * C, f * (VT * (C + F) + 36 * F * C))
        work["conv_before_upsample_out"] = ("hbm", 0, f * (VT * F + P * F))
    else:
        work["conv_before_upsample"] = ("mfma", 2 * P * F * 9 * C, f * P * (C + F))
    px = P
    for o in range(arch.octaves):
        work[f"conv3x3_shuffle2_o{o}"] = ("mfma", 2 * px * 4 * F * 9 * F, f * px * 5 * F)
        px *= 4
    # pixelshuffledirect: one 3x3 conv C -> 3 s^2 stored through pixel_shuffle(s)
    # into the denormalised, cropped image
    work["conv_shuffle_finish"] = ("mfma", 2 * P * 3 * s * s * 9 * C, f * (P * C + 3 * h * s * w * s))
    # nearest+conv: two nearest-2x steps, each with a 3x3 conv F -> F (to 4P
    # and 16P pixels) run as the four output phases' 2x2 convs of the plane
    # before the step (4 taps x F per output instead of 9 x F), then conv_hr
    # at 16P
    work["conv_up1"] = ("mfma", 2 * 4 * P * F * 4 * F, f * (P * F + 4 * P * F))
    work["conv_up2"] = ("mfma", 2 * 16 * P * F * 4 * F, f * (4 * P * F + 16 * P * F))
    work["conv_hr"] = ("mfma", 2 * 16 * P * F * 9 * F, f * 2 * 16 * P * F)
    # pixelshuffle_aux: conv_aux F -> 3 on the VALU with the aux image's
    # denormalisation (the plane in, the aux plane and image out),
    # conv_after_aux 3 -> F; the bicubic resample of the padded input to s x
    # the plane (4 channels)
    Q = (hp * s) * (wp * s)
    work["bicubic"] = ("hbm", 0, f * (4 * P + 4 * Q))
    work["conv_aux"] = ("valu", 2 * P * 3 * 9 * F, f * (P * F + 4 * P + 3 * P))
    work["conv_after_aux"] = ("mfma", 2 * P * F * 27, f * (4 * P + P * F))
    # ... and its bicubic branch through conv_last, composed: a 5x5 conv of the
    # 3 bicubic channels to the 3 outputs over the cropped image (VALU), added
    # into it (the bicubic plane read, the image read and written)
    work["bic_last_add"] = ("valu", 2 * (h * s) * (w * s) * 3 * 75,
                            f * (4 * Q + 2 * 3 * h * s * w * s))
    return work


def traffic_from_profiles(kernel):
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE, WRITE_SIZE),
    if a summary for this kernel is committed under profiles/."""
    p = ROOT / "profiles" / f"{kernel}_traffic.md"
    if not p.exists():
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", p.read_text())
    return float(m.group(1)) if m else None


def cpu_model():
    """The host CPU's model name (/proc/cpuinfo), or "unknown"."""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(M, orc, arch, weights, sample, passes):
    """The oracle (C restatement of the crate's CPU path, OpenMP over the host
    cores) on the same workload: median of `passes` whole-image forwards of a
    `sample` x `sample` input after a 32x32 warm-up."""
    img = M.to_unit(M.input_sinusoids(sample, sample, seed=3))
    x = M.adjust(arch, img)
    warm = M.adjust(arch, M.to_unit(M.input_sinusoids(32, 32, seed=3)))
    orc.forward(arch, weights, 32, 32, warm)
    times = []
    for i in range(passes):
        t0 = time.perf_counter()
        orc.forward(arch, weights, sample, sample, x)
        times.append(time.perf_counter() - t0)
        log(f"bench: cpu pass {i + 1}/{passes}: {times[-1]:.2f} s")
    dt = float(np.median(times))
    out_px = (sample * arch.scale) ** 2
    return {
        "value": round(out_px / dt / 1e6, 5),
        "unit": "Mpix/s",
        "cores": int(orc.lib().orc_threads()),
        "nproc": len(os.sched_getaffinity(0)),
        "cpu_model": cpu_model(),
        "kind": "port",
        "sample": (f"median of {passes} classical-x4 {sample}x{sample}->{sample * arch.scale}x"
                   f"{sample * arch.scale} whole-image forwards (same weights and input), after a"
                   f" 32x32 warm-up; {sum(times):.1f} s of CPU work in total"),
    }


def profile_rows(be, work):
    """{kernel: (total ms, launches)} from the library's event profiler."""
    rows = {}
    for k in work:
        ms, n = be.profile_query(k)
        if n:
            rows[k] = (ms, n)
    return rows


def roofline_of(work, kernel, ms, n, traffic=True):
    """The roofline object for `kernel` from its summed event time over n launches."""
    bound, fl, by = work[kernel]
    avg_s = ms / n / 1e3
    if bound in FLOP_PEAK:
        achieved, peak, unit = fl / avg_s / 1e12, FLOP_PEAK[bound] / 1e12, "TFLOP/s"
    else:
        achieved, peak, unit = by / avg_s / 1e9, HBM_PEAK / 1e9, "GB/s"
    return {"bound": bound, "achieved": round(achieved, 3), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 4),
            "traffic": traffic_from_profiles(kernel) if traffic else None,
            "kernel": kernel, "avg_ms": round(avg_s * 1e3, 4), "launches": n,
            "work_per_launch": fl if bound in FLOP_PEAK else by}


def kernel_table(be, work, steps, rows=None, traffic=True):
    """Per-kernel (launches, avg ms, share, rate) from the library's event
    profiler, logged; returns the rows and the dominant kernel's roofline."""
    if rows is None:
        rows = profile_rows(be, work)
    total_dev = sum(ms for ms, _ in rows.values())
    table = {}
    for k, (ms, n) in sorted(rows.items(), key=lambda kv: -kv[1][0]):
        bound, fl, by = work[k]
        avg = ms / n
        rate = (fl / (avg / 1e3) / 1e12) if bound in FLOP_PEAK else (by / (avg / 1e3) / 1e9)
        unit = "TFLOP/s" if bound in FLOP_PEAK else "GB/s"
        hbm = by / (avg / 1e3) / 1e9
        log(f"  {k:24s} {n:5d} launches {avg:9.4f} ms avg {100 * ms / total_dev:5.1f}% "
            f"{rate:9.2f} {unit}  ({hbm:7.1f} GB/s algorithmic)")
        table[k] = {"launches": n, "avg_ms": round(avg, 4), "rate": round(rate, 2), "unit": unit,
                    "frac": round(rate / (FLOP_PEAK[bound] / 1e12 if bound in FLOP_PEAK else HBM_PEAK / 1e9), 4),
                    "algorithmic_GBps": round(hbm, 1)}
    dom = max(rows, key=lambda k: rows[k][0])
    roofline = roofline_of(work, dom, *rows[dom], traffic=traffic)
    roofline["device_ms_per_step"] = round(total_dev / steps, 3)
    return table, roofline


def bench_rstb(args, pkg):
    """Config 1: one RSTB (6 Swin V2 layers, shifts 0/4, then conv3x3 + 1x1 +
    residual) on an UNPADDED 256x256x180 plane of N(0,1) activations (seed 2),
    1024 windows; weights by the config-0 rules (seed 0). One JSON line with the
    per-kernel rates."""
    M, hip = pkg.model, pkg.hip
    arch = M.Arch(upsampler="pixelshuffle", scale=2, embed=180, heads=6, depths=[6])
    weights = M.make_weights(arch, seed=0)
    hp = wp = 256
    rng = np.random.Generator(np.random.PCG64(2))
    x = rng.standard_normal((hp * wp, arch.embed), dtype=np.float32)
    be = pkg.HipBackend(arch, weights)
    din = hip.DeviceBuffer.from_array(x)
    dout = hip.DeviceBuffer(din.n)
    for _ in range(args.warmup):
        be.rstb_device(0, hp, wp, din.ptr, dout.ptr)
    hip.synchronize()
    # per-kernel pass (events around every launch: the per-kernel table and
    # the dominant kernel's roofline), then the timed calls without events
    work = kernel_work(arch, hp, wp, hp=hp, wp=wp)
    be.profile(True)
    be.profile_reset()
    for _ in range(args.steps):
        be.rstb_device(0, hp, wp, din.ptr, dout.ptr)
    hip.synchronize()
    table, roofline = kernel_table(be, work, args.steps, traffic=False)
    be.profile(False)
    hip.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        be.rstb_device(0, hp, wp, din.ptr, dout.ptr)
    hip.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    assert np.isfinite(dout.download()).all()
    log(f"bench: rstb {args.steps} calls, {ms:.3f} ms per RSTB")
    be.close()
    print(json.dumps({
        "metric": "single-RSTB ms, 256x256x180 fp32 (6 Swin V2 layers + conv3x3 + 1x1 + residual)",
        "value": round(ms, 4), "unit": "ms", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (N(0,1) activations seed 2, random-init weights seed 0)",
        "config": {"workload": "config 1: single RSTB on an unpadded 256x256x180 plane",
                   "windows": (hp // 8) * (wp // 8), "parallelism": "1 GPU"},
        "roofline": roofline, "kernels": table, "kernel_timing": TIMING_NOTE}), flush=True)


def image_workload(M, name, size):
    """(arch, weights, h, w, mean-adjusted input, label, data) of a whole-image
    workload: the headline or BASELINE.json's configs 0, 2 and 3, at their
    sizes, seeds and input generators."""
    if name == "classical-x4":
        arch, seed, h, w = M.classical(4), 3, size, size
        img = M.input_sinusoids(h, w, seed=3)
        data = "synthetic (random-init weights seed 3, config-2 sinusoid input seed 3)"
    elif name == "lightweight-x2":  # config 0
        arch, seed, h, w = M.lightweight(2), 0, 64, 64
        img = M.input_uniform(h, w, seed=1)
        data = "synthetic (random-init weights seed 0, uniform u8 input seed 1)"
    elif name == "classical-x2":  # config 2
        arch, seed, h, w = M.classical(2), 3, 256, 256
        img = M.input_sinusoids(h, w, seed=3)
        data = "synthetic (random-init weights seed 3, sinusoid input seed 3)"
    elif name == "realworld-x4":  # config 3
        arch, seed, h, w = M.realworld(), 4, 480, 640
        img = M.input_texture_dct(h, w, seed=4)
        data = "synthetic (random-init weights seed 4, DCT-quantised texture input seed 4)"
    else:
        raise ValueError(name)
    s = arch.scale
    label = f"{name} {h}x{w}->{h * s}x{w * s}"
    return arch, M.make_weights(arch, seed=seed), h, w, M.adjust(arch, M.to_unit(img)), label, data


TIMING_NOTE = ("kernels: one HIP event pair around each launch on the library's stream, over "
               "forwards launched kernel by kernel; the pair adds about 2 us to each figure, "
               "which is 10-15% of the shortest kernels (profiles/ holds rocprofv3 durations)")


def bench_image(args, pkg, name):
    """A whole-image workload from HBM-resident input to HBM-resident output:
    warm-up, a per-kernel pass (events around every launch), the timed graph
    replays, the replayed output checked bit for bit against an eager forward,
    the dominant kernel's launches timed with events; for the headline also
    the host-buffer path and the CPU baseline. One JSON line."""
    M, hip = pkg.model, pkg.hip
    headline = name == "classical-x4"
    t0 = time.perf_counter()
    arch, weights, h, w, x, label, data = image_workload(M, name, args.size)
    log(f"bench: {label}: weights + input generated in {time.perf_counter() - t0:.1f} s")

    be = pkg.HipBackend(arch, weights)
    dev_name, gfx = pkg.device_info()
    log(f"bench: device {dev_name} {gfx}; uploaded {be.uploaded_bytes() / 2**20:.1f} MiB")
    din = hip.DeviceBuffer.from_array(x)
    s = arch.scale
    shape = (3, h * s, w * s)
    dout = hip.DeviceBuffer(3 * h * s * w * s)
    stream = be.stream()

    if args.copy_probe_mb > 0:
        n = args.copy_probe_mb * 2**20 // 4
        a, b = hip.DeviceBuffer(n), hip.DeviceBuffer(n)
        hip.copy_device(b.ptr, a.ptr, n * 4)
        hip.synchronize()
        a.free()
        b.free()
        log(f"bench: copy probe of {args.copy_probe_mb} MiB done")

    for _ in range(args.warmup):
        be.forward_device(h, w, din.ptr, dout.ptr)
    hip.stream_synchronize(stream)
    log(f"bench: {args.warmup} warm-up steps done")

    # per-kernel pass: K forwards launched kernel by kernel with an event pair
    # around every launch on the library stream (the events cost ~2 us per
    # launch, so this pass is not the one `value` is read from). It names the
    # dominant kernel and gives its launch duration for `roofline`: each launch
    # bracketed by its own pair, as rocprofv3's trace of the same command
    # brackets it (an event pair around that kernel's launches alone read
    # 2-3% longer on the box: the first marker after the preceding kernel
    # then carries that kernel's completion)
    work = kernel_work(arch, h, w)
    be.profile(True)
    be.profile_reset()
    hip.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        be.forward_device(h, w, din.ptr, dout.ptr)
    hip.synchronize()
    prof_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    log(f"bench: per-kernel pass (events around every launch): {prof_ms:.3f} ms/step")
    table, roofline = kernel_table(be, work, args.steps, traffic=headline)
    be.profile(False)
    dom = roofline["kernel"]
    log(f"bench: {dom}: {roofline['avg_ms']:.4f} ms avg, "
        f"{roofline['achieved']} {roofline['unit']} ({100 * roofline['frac']:.1f}% of peak)")

    # timed region: K whole-image forwards as the library runs a repeated
    # call: its launches replayed from the HIP graph it captures the second
    # time the same call comes (the two untimed calls below make sure it has;
    # no events: an event pair cannot bracket one kernel of a graph)
    be.forward_device(h, w, din.ptr, dout.ptr)
    be.forward_device(h, w, din.ptr, dout.ptr)
    hip.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        be.forward_device(h, w, din.ptr, dout.ptr)
    hip.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = wall * 1e3 / args.steps
    out = dout.download(shape)
    value = (h * s) * (w * s) / 1e6 / (ms_per_step / 1e3)
    log(f"bench: {args.steps} timed steps (graph replays), {ms_per_step:.3f} ms/step, "
        f"{value:.3f} output Mpix/s")

    # the timed output, checked: the same input forwarded kernel by kernel into
    # another buffer (a different call, so no graph) must give the replays'
    # output bit for bit; a mismatch fails the run (no JSON line)
    deager = hip.DeviceBuffer(3 * h * s * w * s)
    be.forward_device(h, w, din.ptr, deager.ptr)
    hip.stream_synchronize(stream)
    eager = deager.download(shape)
    deager.free()
    digest = hashlib.sha256(out.tobytes()).hexdigest()[:16]
    if not (np.isfinite(out).all() and np.array_equal(out, eager)):
        log(f"bench: FAILED: the replayed output differs from the eager forward's "
            f"(max |diff| {float(np.nanmax(np.abs(out - eager))):.3e})")
        be.close()
        sys.exit(1)
    log(f"bench: replayed output equals the eager forward's bit for bit (sha256 {digest})")

    # serving figure, reported beside `value` (which stays the one-image rate):
    # the same image twice per step through s2s_forward_device_batch, the two
    # alternating between the context's stream and its second lane, so one
    # image's kernel boundaries overlap the other's kernels; both outputs
    # checked against the one-image output bit for bit
    lanes = None
    if args.lanes:
        din2 = hip.DeviceBuffer.from_array(x)
        douts = [hip.DeviceBuffer(3 * h * s * w * s) for _ in range(2)]
        ins, outs = [din.ptr, din2.ptr], [d.ptr for d in douts]
        for _ in range(3):  # eager, captured per lane, replayed
            be.forward_device_batch(h, w, ins, outs)
        hip.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            be.forward_device_batch(h, w, ins, outs)
        hip.synchronize()
        lane_ms = (time.perf_counter() - t0) * 1e3 / args.steps
        ok = all(np.array_equal(d.download(shape), out) for d in douts)
        for b in [din2] + douts:
            b.free()
        if not ok:
            log("bench: FAILED: a two-lane output differs from the one-image forward's")
            be.close()
            sys.exit(1)
        lanes = {"images_per_step": 2, "ms_per_step": round(lane_ms, 4),
                 "ms_per_image": round(lane_ms / 2, 4),
                 "mpix_s": round(2 * (h * s) * (w * s) / 1e3 / lane_ms, 4),
                 "outputs_equal_one_image_forward": True}
        log(f"bench: two lanes (s2s_forward_device_batch, 2 images per step): {lane_ms:.3f} ms per "
            f"step, {lanes['mpix_s']:.3f} output Mpix/s")

    win = arch.window
    result = {
        "metric": METRIC if headline else f"output Mpix/s {label} fp32 @1 GPU",
        "value": round(value, 4), "unit": "Mpix/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": data,
        "config": {"workload": f"{label} whole-image forward",
                   "embed": arch.embed, "depths": arch.depths, "heads": arch.heads,
                   "upsampler": arch.upsampler, "window": win,
                   "padded_plane": [(h // win + 1) * win, (w // win + 1) * win],
                   "parallelism": "1 GPU"},
        "roofline": roofline,
        "kernels": table,
        "kernel_timing": TIMING_NOTE,
        "output_check": {"replay_equals_eager": True, "sha256_16": digest},
    }
    if lanes:
        result["two_lane_serving"] = lanes
    if headline:
        # the crate's own boundary hands over host slices: s2s_forward uploads
        # the input, runs, downloads the output (PCIe included); reported, never
        # `value`. The crate's backend returns a new Vec per forward, so the
        # first figure takes a fresh output array per call (its first-touch
        # cost included); the second reuses one.
        xh = np.ascontiguousarray(x)
        be.forward(h, w, xh)
        host_ms, host_mean = {}, {}
        for mode in ("fresh", "reused"):
            keep = np.empty(shape, np.float32) if mode == "reused" else None
            per = []
            for _ in range(max(args.steps, 10)):
                t0 = time.perf_counter()
                be.forward(h, w, xh, out=keep)
                per.append((time.perf_counter() - t0) * 1e3)
            # the median of at least 10 synchronous calls (the crate's wall per
            # image), the mean beside it
            host_ms[mode] = float(np.median(per))
            host_mean[mode] = float(np.mean(per))
        log(f"bench: host-buffer path (s2s_forward, PCIe included): {host_ms['fresh']:.3f} ms "
            f"({(h * s) * (w * s) / 1e3 / host_ms['fresh']:.3f} output Mpix/s, "
            f"{100 * (host_ms['fresh'] / ms_per_step - 1):.1f}% over the device-resident step) with a "
            f"fresh output per call; {host_ms['reused']:.3f} ms into a reused one")
        result["host_path_mpix_s"] = round((h * s) * (w * s) / 1e3 / host_ms["fresh"], 3)
        result["host_path_ms"] = round(host_ms["fresh"], 4)
        result["host_path_reused_out_ms"] = round(host_ms["reused"], 4)
        result["host_path_timing"] = (f"median of {max(args.steps, 10)} synchronous s2s_forward calls "
                                      f"(means {host_mean['fresh']:.4f} and {host_mean['reused']:.4f} ms)")
    be.close()
    if headline and not args.no_cpu:
        orc = ge._load_oracle()
        log(f"bench: cpu baseline on {orc.lib().orc_threads()} threads ...")
        result["cpu_baseline"] = cpu_baseline(M, orc, arch, weights, args.cpu_sample,
                                              args.cpu_passes)
        log(f"bench: cpu {result['cpu_baseline']}")
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)


class _TimedBackend:
    """`Backend` over the HIP context for the tile loop, adding each call's
    wall time."""

    def __init__(self, be):
        self.be, self.ms = be, 0.0

    def forward(self, h, w, x):
        t0 = time.perf_counter()
        out = self.be.forward(h, w, x)
        self.ms += (time.perf_counter() - t0) * 1e3
        return out


def bench_tiled(args, pkg):
    """Config 4: compressed x4 (pixelshuffle_aux), 1024x1024 -> 4096x4096 in
    256-pixel tiles with 64 of context, through the crate's tile loop
    (run_tiled) over the host-buffer entry s2s_forward, one tile after another
    on one GPU, as the crate's --tile path runs it (PCIe included per tile).
    `value` is output Mpix/s of whole tiled images. One JSON line, with the
    per-kernel table of one profiled tiled run (work averaged over the tiles'
    planes)."""
    M, T = pkg.model, pkg.tiling
    arch = M.compressed()
    size, tile, pad = 1024, 256, 64
    t0 = time.perf_counter()
    weights = M.make_weights(arch, seed=5)
    img = M.to_unit(M.input_texture_dct(size, size, seed=5))
    log(f"bench: weights + input generated in {time.perf_counter() - t0:.1f} s")
    be = pkg.HipBackend(arch, weights)
    rec = []

    class Rec:
        def forward(self, h, w, x):
            rec.append((h, w))
            return be.forward(h, w, x)

    for _ in range(max(args.warmup, 1)):
        T.run_tiled(arch, Rec(), img, tile, pad)
    tiles = rec[:len(rec) // max(args.warmup, 1)]
    log(f"bench: {args.warmup} warm-up tiled runs done ({len(tiles)} tiles)")
    # per-kernel pass: one tiled run with events around every launch; each
    # kernel's work per launch is the average over the tiles' planes
    work = {}
    for h, w in tiles:
        for k, (bound, fl, by) in kernel_work(arch, h, w).items():
            b0, f0, y0 = work.get(k, (bound, 0, 0))
            work[k] = (bound, f0 + fl / len(tiles), y0 + by / len(tiles))
    be.profile(True)
    be.profile_reset()
    T.run_tiled(arch, be, img, tile, pad)
    table, roofline = kernel_table(be, work, 1)
    be.profile(False)
    tb = _TimedBackend(be)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        out = T.run_tiled(arch, tb, img, tile, pad)
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    assert out.shape == (3, size * 4, size * 4) and np.isfinite(out).all()
    value = (size * 4) ** 2 / 1e6 / (ms / 1e3)
    log(f"bench: {args.steps} tiled runs, {ms:.2f} ms per image ({tb.ms / args.steps:.2f} ms in "
        f"s2s_forward), {value:.3f} output Mpix/s")
    # serving figure, reported beside `value` (which stays the crate's
    # one-tile-after-another loop): the same tile loop with the image's crops
    # in one s2s_forward_batch call, alternating between the context's two
    # lanes, so one tile's upload/download and kernel boundaries overlap the
    # other lane's kernels; the image checked against the sequential one bit
    # for bit
    batched = None
    if args.lanes:
        for _ in range(2):  # each lane captures, then replays
            T.run_tiled(arch, be, img, tile, pad, batch=True)
        t0 = time.perf_counter()
        for _ in range(args.steps):
            out_b = T.run_tiled(arch, be, img, tile, pad, batch=True)
        ms_b = (time.perf_counter() - t0) * 1e3 / args.steps
        if not np.array_equal(out_b, out):
            log("bench: FAILED: the batched tiled image differs from the sequential one")
            be.close()
            sys.exit(1)
        batched = {"ms_per_image": round(ms_b, 3),
                   "mpix_s": round((size * 4) ** 2 / 1e6 / (ms_b / 1e3), 4),
                   "image_equals_sequential": True}
        log(f"bench: batched tile loop (s2s_forward_batch over two lanes): {ms_b:.2f} ms per image, "
            f"{batched['mpix_s']:.3f} output Mpix/s")
    be.close()
    print(json.dumps({
        "metric": "output Mpix/s compressed-x4 1024x1024->4096x4096 tiled (256 + 64 context) fp32 @1 GPU",
        "value": round(value, 4), "unit": "Mpix/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 3), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (random-init weights seed 5, DCT-quantised texture input seed 5)",
        "config": {"workload": "config 4: compressed x4 1024x1024 in 16 tiles of 256 + 64 context "
                               "through run_tiled over s2s_forward (host buffers, PCIe included)",
                   "tiles": [list(t) for t in tiles], "parallelism": "1 GPU"},
        "ms_in_forward_per_step": round(tb.ms / args.steps, 3),
        "roofline": roofline, "kernels": table, "kernel_timing": TIMING_NOTE,
        "two_lane_tiles": batched,
        "cpu_baseline": None}), flush=True)


def bench_copy_ceiling(args, pkg):
    """The HBM streaming ceiling the memory-bound kernels are read against: the
    runtime's own device-to-device copy kernel (hipMemcpy), timed with events
    over `steps` copies enqueued back to back on the null stream at each size;
    bytes moved = 2 x size (read + write).
    The sizes span the memory-bound kernels' traffic at the headline workload
    (50 MB planes to the 213 MB of the Winograd output transform) and a 1 GiB
    copy, larger than the 256 MB last-level cache. One JSON line."""
    hip = pkg.hip
    res = {}
    for mib in (16, 50, 100, 200, 400, 1024):
        n = mib * 2**20 // 4
        a, b = hip.DeviceBuffer(n), hip.DeviceBuffer(n)
        for _ in range(max(args.warmup, 1)):
            hip.copy_device(b.ptr, a.ptr, n * 4)
        hip.synchronize()
        e0, e1 = hip.Event(), hip.Event()
        e0.record(0)
        for _ in range(args.steps):
            hip.copy_device_async(b.ptr, a.ptr, n * 4, 0)
        e1.record(0)
        e1.synchronize()
        ms = e0.elapsed_ms(e1) / args.steps
        gbps = 2 * n * 4 / (ms / 1e3) / 1e9
        res[f"{mib} MiB"] = {"avg_ms": round(ms, 4), "GBps": round(gbps, 1),
                             "frac_of_8TBps": round(gbps / (HBM_PEAK / 1e9), 4)}
        log(f"bench: copy {mib:5d} MiB: {ms:.4f} ms, {gbps:.1f} GB/s "
            f"({100 * gbps / (HBM_PEAK / 1e9):.1f}% of 8 TB/s)")
        a.free()
        b.free()
    print(json.dumps({"metric": "device-to-device copy GB/s (read + write bytes) @1 GPU",
                      "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
                      "higher_is_better": True, "dtype": "f32", "data": "uninitialised buffers",
                      "config": {"workload": "hipMemcpyAsync device-to-device (the runtime's "
                                             "copy kernel), null stream, event-timed"},
                      "sizes": res}), flush=True)


def bench_mfma_peak(args, pkg):
    """The fp32 matrix ceiling the MFMA-bound kernels are read against, beside
    the 157.3 TFLOP/s spec figure: the library's probe kernel (one 512-thread
    workgroup per CU, every wave issuing independent v_mfma_f32_16x16x4f32 and
    nothing else), `steps` launches timed with events, at two loop lengths
    (the longer one's rate is the ceiling; the pair shows the launch is
    amortised). The implied shader clock is the rate over 64 FLOPs per cycle
    per SIMD. One JSON line."""
    res = {}
    for iters in (5000, 40000):
        ms, tf, ghz = pkg.abi.mfma_peak(iters, max(args.steps, 1))
        res[str(iters)] = {"ms_per_launch": round(ms, 4), "TFLOPs": round(tf, 2),
                           "frac_of_spec": round(tf * 1e12 / MFMA_FP32_PEAK, 4),
                           "implied_clock_GHz": round(ghz, 3)}
        log(f"bench: mfma peak probe, {4 * iters} MFMAs per wave: {ms:.3f} ms, {tf:.2f} TFLOP/s "
            f"({100 * tf * 1e12 / MFMA_FP32_PEAK:.1f}% of 157.3), implied clock {ghz:.3f} GHz")
    print(json.dumps({"metric": "fp32 MFMA TFLOP/s under pure MFMA load @1 GPU", "unit": "TFLOP/s",
                      "n_gpus": 1, "steps": args.steps, "higher_is_better": True, "dtype": "f32",
                      "data": "register operands",
                      "config": {"workload": "k_mfma_peak: one 512-thread workgroup per CU, 4 independent "
                                             "v_mfma_f32_16x16x4f32 per loop iteration per wave"},
                      "loops": res}), flush=True)


WORKLOADS = ["classical-x4", "rstb", "lightweight-x2", "classical-x2", "realworld-x4",
             "compressed-x4-tiled", "copy-ceiling", "mfma-peak"]


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--size", type=int, default=256, help="classical-x4 input side")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-sample", type=int, default=256)
    ap.add_argument("--cpu-passes", type=int, default=3)
    ap.add_argument("--workload", choices=WORKLOADS, default="classical-x4",
                    help="classical-x4: the BASELINE metric (default); rstb: config 1's "
                         "single-RSTB micro-bench; lightweight-x2, classical-x2, realworld-x4: "
                         "configs 0, 2, 3 whole-image; compressed-x4-tiled: config 4; "
                         "copy-ceiling: the runtime's device copy at several sizes; "
                         "mfma-peak: the fp32 matrix rate under pure MFMA load")
    ap.add_argument("--lanes", type=int, default=1, choices=[0, 1],
                    help="also time two images per step through the two-lane batched entry "
                         "(reported as two_lane_serving; value stays the one-image rate); with "
                         "compressed-x4-tiled, the tile loop over s2s_forward_batch "
                         "(two_lane_tiles)")
    ap.add_argument("--copy-probe-mb", type=int, default=0,
                    help="before the warm-up, one device-to-device copy of this many MiB: the "
                         "plain copy kernel of known size that scales rocprofv3's FETCH_SIZE / "
                         "WRITE_SIZE counters to bytes")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this backend runs a whole image on one device and has "
              "no multi-GPU path (images and tiles are independent, so several GPUs would each "
              "take their share of them); run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    pkg = ge.load_package()
    if args.workload == "rstb":
        bench_rstb(args, pkg)
    elif args.workload == "compressed-x4-tiled":
        bench_tiled(args, pkg)
    elif args.workload == "copy-ceiling":
        bench_copy_ceiling(args, pkg)
    elif args.workload == "mfma-peak":
        bench_mfma_peak(args, pkg)
    else:
        bench_image(args, pkg, args.workload)


if __name__ == "__main__":
    main()
