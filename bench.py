"""Benchmark of the MI355X HTDemucs backend (one JSON line on stdout).

Workload ("config 3"): full htdemucs separation of a
60 s stereo 44.1 kHz synthetic mix, fp32, random-init weights (seed 0), 7.8 s
segments at overlap 0.25 batched 8 chunks per launch, shifts = 0. One step =
one separation from host f32 samples in to host f32 stems out (dmx_separate:
the mix upload, the chunk loop on the GPU and the stem readback are all inside
the clock, as the metric defines it).
value = x-realtime = audio seconds / wall seconds over the timed steps.

Beside it: the same separation with mix and stems resident in HBM
(dmx_separate_device); the same workload driven through the SegmentForward
entry points (dmx_forward_start / collect, one group queued ahead, the chunk
loop on the host as the reference's pipeline runs it); the cross-attention
kernel's TFLOP/s at the model's shape (Q 2688 vs K/V 1344 and Q 1344 vs K/V
2688, a cross layer's two directions, in one launch; 8 heads x 64, batch 8)
and its roofline fraction against the fp32 MFMA peak, measured with HIP events
on the launch stream; and the restated reference CPU backend (oracle/) timed
on this host on the same config-3 separation.
"""
import argparse
import ctypes
import importlib.util
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
PACKAGE_DIR = ROOT / "demucs-wgpu_amd"

FP32_MFMA_PEAK_TFLOPS = 157.3  # MI355X dense fp32 matrix peak (datasheet)


def load_package():
    name = "demucs_wgpu_amd"
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, PACKAGE_DIR / "__init__.py",
                                                  submodule_search_locations=[str(PACKAGE_DIR)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def attention_roofline(pkg, torch, batch: int, iters: int, precision: int = 0, planes: bool = False):
    """Average duration of the fused cross-attention kernel on a cross
    layer's work: both directions of the model's cross shape in one launch
    (Lq = 2688 spectral tokens vs Lk = 1344 waveform tokens, and Lq = 1344 vs
    Lk = 2688; the runner issues them as two concurrent launches on the branch
    streams), timed with events on the stream it is launched on.
    Returns (ms per launch, algorithmic flops per launch)."""
    from demucs_wgpu_amd import _native
    lib = _native.load()
    assert lib.dmx_op_set_precision(precision) == 0, lib.dmx_last_error()
    heads, D = 8, 512
    (lq0, lk0), (lq1, lk1) = (2688, 1344), (1344, 2688)
    t = {}
    for name, lq, lk in (("0", lq0, lk0), ("1", lq1, lk1)):
        t["q" + name] = torch.randn(batch, lq, D, device="cuda")
        t["k" + name] = torch.randn(batch, lk, D, device="cuda")
        t["v" + name] = torch.randn(batch, lk, D, device="cuda")
        t["o" + name] = torch.empty(batch, lq, D, device="cuda")
    stream = torch.cuda.current_stream()
    P = lambda x: ctypes.c_void_p(x.data_ptr())
    sp = ctypes.c_void_p(stream.cuda_stream)
    if planes:
        # The three-plane kernel reads K and V as planes, which the runner's
        # in-projection writes; here they are made once, outside the timing.
        for name, lk in (("0", lk0), ("1", lk1)):
            ldvt = (lk + 31) // 32 * 32
            t["kp" + name] = torch.empty(3 * batch * lk * D, dtype=torch.int16, device="cuda")
            t["vt" + name] = torch.empty(3 * batch * D * ldvt, dtype=torch.int16, device="cuda")
            assert lib.dmx_op_kv_planes(sp, P(t["k" + name]), P(t["v" + name]), batch, heads, lk,
                                        P(t["kp" + name]), P(t["vt" + name])) == 0, lib.dmx_last_error()
        fn = lib.dmx_op_attention_pair_planes
        args = (sp, P(t["q0"]), P(t["kp0"]), P(t["vt0"]), P(t["o0"]), lq0, lk0, P(t["q1"]), P(t["kp1"]),
                P(t["vt1"]), P(t["o1"]), lq1, lk1, batch, heads, ctypes.c_float(0.125))
    else:
        fn = lib.dmx_op_attention_pair
        args = (sp, P(t["q0"]), P(t["k0"]), P(t["v0"]), P(t["o0"]), lq0, lk0,
                P(t["q1"]), P(t["k1"]), P(t["v1"]), P(t["o1"]), lq1, lk1, batch, heads, ctypes.c_float(0.125))
    for _ in range(3):
        assert fn(*args) == 0, lib.dmx_last_error()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(iters):
        fn(*args)
    end.record(stream)
    end.synchronize()
    ms = start.elapsed_time(end) / iters
    flops = 4.0 * batch * D * (lq0 * lk0 + lq1 * lk1)  # QK^T + PV, 2 flops per MAC, both problems
    return ms, flops


TRAFFIC_SUMMARY = ROOT / "profiles" / "attention_cross_b8_traffic.md"
ATTENTION_SOURCE = PACKAGE_DIR / "csrc" / "attention.hip"


def measured_traffic():
    """HBM bytes per launch of the roofline kernel from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary (copy-kernel calibrated), with
    where it comes from. The summary records the sha256 of the kernel source
    it measured; when attention.hip has changed since, the figure is stale and
    the traffic is reported as null."""
    import hashlib
    fields = {}
    try:
        for line in TRAFFIC_SUMMARY.read_text().splitlines():
            if ":" in line and not line.startswith((" ", "|", "#")):
                k, v = line.split(":", 1)
                fields[k.strip()] = v.strip()
    except OSError:
        return None, "no traffic summary"
    current = hashlib.sha256(ATTENTION_SOURCE.read_bytes()).hexdigest()
    if fields.get("source_sha256") != current:
        return None, f"{TRAFFIC_SUMMARY.name} measured another attention.hip (sha256 {fields.get('source_sha256')})"
    return int(fields["traffic_bytes_per_launch"]), (
        f"{TRAFFIC_SUMMARY.relative_to(ROOT)}: rocprofv3 FETCH_SIZE + WRITE_SIZE per dispatch, scaled by a 256 MiB "
        f"copy's counters; measured on attention.hip sha256 {current[:16]}, the source built here")


def copy_calibration(torch, mib: int = 256, iters: int = 5):
    """A plain device copy of known size: rocprofv3's FETCH_SIZE / WRITE_SIZE for
    this kernel over `mib` MiB read and written gives the counters' scale."""
    n = mib * (1 << 20) // 4
    src = torch.ones(n, device="cuda")
    dst = torch.empty(n, device="cuda")
    for _ in range(iters):
        dst.copy_(src)
    torch.cuda.synchronize()
    return mib


def transformer_flops(d=512, ff=2048, lf=2688, lt=1344, layers=5):
    """Algorithmic FLOPs of the cross-transformer stack per batch element
    (projections, QK^T and PV, FFN; 2 flops per MAC): self layers at even
    indices, cross layers at odd ones, both branches."""
    def self_layer(n):
        return 2 * n * d * 3 * d + 4 * n * n * d + 2 * n * d * d + 4 * n * d * ff

    def cross_layer(nq, nk):
        return 2 * nq * d * d + 2 * nk * d * 2 * d + 4 * nq * nk * d + 2 * nq * d * d + 4 * nq * d * ff
    total = 0
    for i in range(layers):
        total += (self_layer(lf) + self_layer(lt)) if i % 2 == 0 else (cross_layer(lf, lt) + cross_layer(lt, lf))
    return float(total)


def config2_transformer(pkg, torch, batch=8, iters=5):
    """Config 2: the 5-layer cross-transformer alone on N(0, 1) activations,
    2688 frequency tokens (8 x 336) and 1344 time tokens, Xavier-init."""
    cfg = pkg.Config()
    runner = pkg.Runner(pkg.xavier_transformer_init(0, cfg), cfg)
    g = torch.Generator(device="cuda").manual_seed(0)
    x = torch.randn((batch, 512, 8, 336), device="cuda", generator=g)
    xt = torch.randn((batch, 512, 1344), device="cuda", generator=g)
    ox, oxt = torch.empty_like(x), torch.empty_like(xt)
    torch.cuda.synchronize()
    run = lambda: runner.crosstransformer_device(x.data_ptr(), xt.data_ptr(), batch, 8, 336, 1344, ox.data_ptr(),
                                                 oxt.data_ptr())
    run()
    runner.synchronize()
    t0 = time.perf_counter()
    for _ in range(iters):
        run()
    runner.synchronize()
    ms = 1000.0 * (time.perf_counter() - t0) / iters
    flops = transformer_flops() * batch
    return {"batch": batch, "ms": round(ms, 3), "tflops": round(flops / (ms * 1e-3) / 1e12, 2),
            "flops_per_call": flops, "dtype": "f32"}


def config4_bag(pkg, torch, seconds=180.0, batch_chunks=8):
    """Config 4: four random-init networks (seeds 1-4), identity bag, shifts=1,
    180 s synthetic mix resident in HBM; then StemSelection::Some([vocals])."""
    cfg = pkg.Config()
    runners = [pkg.Runner(pkg.random_init(seed, cfg), cfg) for seed in (1, 2, 3, 4)]
    mix = pkg.signals.synthetic_mix(0, seconds)
    samples = mix.shape[1]
    d_mix = torch.from_numpy(mix).cuda()
    d_stems = torch.empty((cfg.sources, 2, samples), device="cuda")
    bag = np.eye(4, cfg.sources, dtype=np.float32)
    opts = pkg.SeparateOptions(shifts=1, overlap=0.25, batch_chunks=batch_chunks).to_c()
    lib = pkg._native.load()
    handles = (ctypes.c_void_p * 4)(*[r.handle for r in runners])

    def sep(wanted):
        mask = None if wanted is None else (ctypes.c_uint8 * 4)(*wanted)
        rc = lib.dmx_separate_device(handles, bag.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), 4, mask,
                                     ctypes.c_void_p(d_mix.data_ptr()), samples, cfg.samplerate, ctypes.byref(opts),
                                     pkg._native.PROGRESS(), None, ctypes.c_void_p(d_stems.data_ptr()))
        if rc != 0:
            raise RuntimeError(pkg._native.last_error())
        runners[0].synchronize()
        torch.cuda.synchronize()

    out = {}
    for name, wanted in (("all_stems", None), ("vocals_only", (0, 0, 0, 1))):
        sep(wanted)
        t0 = time.perf_counter()
        sep(wanted)
        s = time.perf_counter() - t0
        out[name] = {"x_realtime": round(seconds / s, 2), "ms": round(1000.0 * s, 2)}
    out["workload"] = (f"{seconds:g} s mix, 4 networks (seeds 1-4), identity bag, shifts=1, overlap 0.25, "
                       f"{batch_chunks} chunks per launch, fp32, mix and stems resident in HBM")
    return out


def config5_bf16(pkg, torch, batch=32, iters=3, check=2):
    """Config 5: the full forward with bf16-MFMA contractions on 32 segments of
    N(0, 0.1^2) noise (seed-7 weights); per-stem SNR of `check` of them against
    the fp32 oracle on the host."""
    cfg = pkg.Config()
    w = pkg.random_init(7, cfg)
    runner = pkg.Runner(w, cfg, precision=pkg.PRECISION_BF16)
    L = cfg.training_length
    mix = pkg.signals.gaussian_segments(7, batch, L)
    d_mix = torch.from_numpy(mix).cuda()
    d_out = torch.empty((batch, cfg.sources, 2, L), device="cuda")
    lib = pkg._native.load()

    def fwd():
        rc = lib.dmx_forward_device(runner.handle, ctypes.c_void_p(d_mix.data_ptr()), batch, 2, L,
                                    ctypes.c_void_p(d_out.data_ptr()))
        if rc != 0:
            raise RuntimeError(pkg._native.last_error())
    fwd()
    runner.synchronize()
    t0 = time.perf_counter()
    for _ in range(iters):
        fwd()
    runner.synchronize()
    s = (time.perf_counter() - t0) / iters
    sys.path.insert(0, str(ROOT))
    from oracle import binding as oracle
    ref = oracle.Model(w, cfg).forward(mix[:check])
    got = d_out[:check].cpu().numpy()
    snr = min(10.0 * np.log10(np.sum(ref[:, s_].astype(np.float64) ** 2) /
                              max(np.sum((ref[:, s_].astype(np.float64) - got[:, s_]) ** 2), 1e-30))
              for s_ in range(cfg.sources))
    return {"batch": batch, "ms": round(1000.0 * s, 2), "x_realtime": round(batch * L / cfg.samplerate / s, 2),
            "min_stem_snr_db_vs_fp32_oracle": round(float(snr), 2), "snr_checked_segments": check,
            "dtype": "bf16 MFMA inputs, f32 accumulate/softmax/norms/output"}


def host_cpu():
    """(threads the oracle may use, model name) of this host."""
    model = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return os.cpu_count(), model


def cpu_baseline(pkg, seconds: float, batch_chunks: int, repeats: int = 3):
    """The restated reference CPU backend (oracle/, OpenMP on every host core)
    on the headline workload: the config-3 separation of the same mix with
    the same weights, after one warm-up forward; median of `repeats`. One
    7.8 s segment forward (config 1) is timed beside it."""
    sys.path.insert(0, str(ROOT))
    from oracle import binding as oracle
    cfg = pkg.Config()
    weights = pkg.random_init(0, cfg)
    model = oracle.Model(weights, cfg)
    seg = pkg.signals.gaussian_segments(0, 1, cfg.training_length)
    model.forward(seg)  # warm-up: threads, pages, caches
    mix = pkg.signals.synthetic_mix(0, seconds)
    opts = pkg.SeparateOptions(shifts=0, overlap=0.25, batch_chunks=batch_chunks)
    times = []
    for _ in range(repeats):
        t0 = time.perf_counter()
        oracle.separate([model], mix[0], mix[1], cfg.samplerate, opts)
        times.append(time.perf_counter() - t0)
    t = float(np.median(times))
    t0 = time.perf_counter()
    model.forward(seg)
    t1 = time.perf_counter() - t0
    seg_s = cfg.training_length / cfg.samplerate
    nproc, cpu_model = host_cpu()
    return {"value": round(seconds / t, 4), "unit": "x-realtime", "cores": oracle.threads(), "kind": "port",
            "sample": f"config 3: separation of the {seconds:g} s mix (11 chunks of 7.8 s, groups of {batch_chunks}), "
                      f"restated reference CPU backend, median of {repeats} after a warm-up forward: {t:.2f} s each",
            "host": {"nproc": nproc, "cpu_model": cpu_model},
            "config1_forward": {"x_realtime": round(seg_s / t1, 4), "s": round(t1, 3)}}


def segment_forward_path(pkg, runner, mix, batch_chunks: int, ref_stems, repeats: int = 3):
    """Config 3 driven through SegmentForward (dmx_forward_start / collect), as
    the reference's pipeline drives its runner (crates/demucs-core/src/demucs/
    pipeline.rs:380-515, :584-619; streaming.rs:296-400): the host normalises
    the mix, cuts centred zero-padded chunks, queues group n + 1 before it
    collects group n, and overlap-adds on the host (numpy here). Returns the
    best of `repeats` and the SNR of its stems against dmx_separate's."""
    cfg = runner.config
    seg = cfg.training_length
    stride = int(0.75 * seg)
    samples = mix.shape[1]
    half = seg // 2
    weight = np.concatenate([np.arange(1, half + 1), np.arange(seg - half, 0, -1)]).astype(np.float32)
    weight /= max(float(weight.max()), 1.0)
    ref = (mix[0].astype(np.float64) + mix[1]) / 2.0
    mean = np.float32(ref.mean())
    std = np.float32(np.sqrt(ref.var(ddof=1))) + np.float32(1e-8)
    starts = list(range(0, samples, stride))

    def run():
        norm = (mix - mean) / std
        acc = np.zeros((cfg.sources, 2, samples), np.float32)
        sum_w = np.zeros(samples, np.float32)
        groups = [starts[i:i + batch_chunks] for i in range(0, len(starts), batch_chunks)]
        in_calls = 0.0

        def chunks(g):
            x = np.zeros((len(g), 2, seg), np.float32)
            for j, s0 in enumerate(g):
                n = min(samples - s0, seg)
                off = (seg - n) // 2
                lo = s0 - off
                a, b = max(lo, 0), min(lo + seg, samples)
                x[j, :, a - lo:b - lo] = norm[:, a:b]
            return x

        t0 = time.perf_counter()
        pending = runner.start(chunks(groups[0]))
        in_calls += time.perf_counter() - t0
        for gi, g in enumerate(groups):
            nxt = None
            if gi + 1 < len(groups):
                x = chunks(groups[gi + 1])
                t1 = time.perf_counter()
                nxt = runner.start(x)
                in_calls += time.perf_counter() - t1
            t1 = time.perf_counter()
            out = runner.collect(pending)
            in_calls += time.perf_counter() - t1
            for j, s0 in enumerate(g):
                n = min(samples - s0, seg)
                trim = (seg - n) // 2
                acc[:, :, s0:s0 + n] += weight[:n] * out[j, :, :, trim:trim + n]
                sum_w[s0:s0 + n] += weight[:n]
            pending = nxt
        stems = acc / sum_w * std + mean
        return stems, in_calls

    run()
    best = None
    for _ in range(repeats):
        t0 = time.perf_counter()
        stems, in_calls = run()
        wall = time.perf_counter() - t0
        if best is None or wall < best[0]:
            best = (wall, in_calls)
    err = stems.astype(np.float64) - ref_stems
    snr = 10.0 * np.log10(np.sum(ref_stems.astype(np.float64) ** 2) / max(float(np.sum(err * err)), 1e-30))
    audio_s = samples / cfg.samplerate
    return {"x_realtime": round(audio_s / best[0], 2), "ms": round(1000.0 * best[0], 2),
            "ms_in_start_collect": round(1000.0 * best[1], 2),
            "snr_db_vs_dmx_separate": round(float(snr), 1),
            "note": f"{len(starts)} chunks in groups of {batch_chunks}, group n+1 started before group n is "
                    "collected; normalisation, chunking and overlap-add in numpy on the host; best of "
                    f"{repeats} after a warm-up"}


def profile_workload(pkg, torch, args):
    """One workload alone, for rocprofv3 (kernel trace, memory-copy trace or
    counters): `--warmup` untimed and `--steps` timed calls, then the copy
    that calibrates FETCH_SIZE / WRITE_SIZE. Returns the wall time per call."""
    cfg = pkg.Config()
    lib = pkg._native.load()
    if args.profile == "bf16":
        batch = 32
        runner = pkg.Runner(pkg.random_init(7, cfg), cfg, precision=pkg.PRECISION_BF16)
        L = cfg.training_length
        d_mix = torch.from_numpy(pkg.signals.gaussian_segments(7, batch, L)).cuda()
        d_out = torch.empty((batch, cfg.sources, 2, L), device="cuda")

        def call():
            rc = lib.dmx_forward_device(runner.handle, ctypes.c_void_p(d_mix.data_ptr()), batch, 2, L,
                                        ctypes.c_void_p(d_out.data_ptr()))
            if rc != 0:
                raise RuntimeError(pkg._native.last_error())
        what = f"config 5: bf16 forward of {batch} segments (dmx_forward_device)"
    else:
        runner = pkg.Runner(pkg.random_init(0, cfg), cfg, precision=fp32_precision(pkg, args))
        mix = pkg.signals.synthetic_mix(0, args.seconds)
        samples = mix.shape[1]
        opts = pkg.SeparateOptions(shifts=0, overlap=0.25, batch_chunks=args.batch_chunks)
        if args.profile == "host":
            left, right = np.ascontiguousarray(mix[0]), np.ascontiguousarray(mix[1])

            def call():
                pkg.separate_runners([runner], left, right, cfg.samplerate, opts)
            what = f"config 3: {args.seconds:g} s separation, host arrays in and out (dmx_separate)"
        else:
            d_mix = torch.from_numpy(mix).cuda()
            d_stems = torch.empty((cfg.sources, 2, samples), device="cuda")
            c_opts = opts.to_c()
            handles = (ctypes.c_void_p * 1)(runner.handle)

            def call():
                rc = lib.dmx_separate_device(handles, None, 1, None, ctypes.c_void_p(d_mix.data_ptr()), samples,
                                             cfg.samplerate, ctypes.byref(c_opts), pkg._native.PROGRESS(), None,
                                             ctypes.c_void_p(d_stems.data_ptr()))
                if rc != 0:
                    raise RuntimeError(pkg._native.last_error())
            what = f"config 3: {args.seconds:g} s separation, mix and stems in HBM (dmx_separate_device)"
    for _ in range(args.warmup):
        call()
    runner.synchronize()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        call()
    runner.synchronize()
    torch.cuda.synchronize()
    ms = 1000.0 * (time.perf_counter() - t0) / max(1, args.steps)
    mib = copy_calibration(torch)
    return {"profile": args.profile, "workload": what, "warmup": args.warmup, "steps": args.steps,
            "ms_per_call": round(ms, 3), "copy_calibration_mib": mib}


BF16_MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense bf16


def planes_attention(args) -> bool:
    """Whether the fp32 runs use the three-plane attention kernel (the default
    precision, unless the DMX_ATT_PLANES=0 tuning switch keeps fp32 MFMA)."""
    return args.precision == "fp32" and os.environ.get("DMX_ATT_PLANES", "1") != "0"


def attention_roofline_record(args, attn_ms, attn_tflops, traffic, traffic_source):
    """The roofline object of the cross-attention launch. The three-plane
    kernel's algorithm is six bf16 plane products per fp32 multiply-add on the
    bf16 matrix cores, so its achieved rate is 6x the fp32-equivalent rate,
    against the bf16 dense peak; the fp32-MFMA kernel's is the fp32 rate
    against the fp32 peak."""
    launch = "dmx_op_attention_pair_planes" if planes_attention(args) else "dmx_op_attention_pair"
    shape = (f"sum of 4*B*Lq*Lk*512 flops over (Lq, Lk) = (2688, 1344) and (1344, 2688), B={args.batch_chunks}, "
             f"both directions in one launch ({launch}); avg {attn_ms:.3f} ms per launch")
    if planes_attention(args):
        achieved = 6.0 * attn_tflops
        return {"bound": "mfma", "achieved": round(achieved, 2), "peak": BF16_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(achieved / BF16_MFMA_PEAK_TFLOPS, 4), "traffic": traffic,
                "traffic_source": traffic_source,
                "kernel": "attention_x3_kernel (fused cross-attention, fp32-accurate: Q, K, V and P as three bf16 "
                          "planes, six plane products per multiply-add on v_mfma_f32_32x32x16_bf16)",
                "per_launch": "6 x (" + shape + ")",
                "fp32_equivalent": {"tflops": round(attn_tflops, 2),
                                    "frac_of_fp32_peak": round(attn_tflops / FP32_MFMA_PEAK_TFLOPS, 4)}}
    return {"bound": "mfma", "achieved": round(attn_tflops, 2), "peak": FP32_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(attn_tflops / FP32_MFMA_PEAK_TFLOPS, 4), "traffic": traffic,
            "traffic_source": traffic_source, "kernel": "attention_kernel (fused cross-attention, fp32 MFMA)",
            "per_launch": shape}


def fp32_precision(pkg, args):
    """The runner precision of the fp32 workloads (--precision)."""
    return pkg.PRECISION_FP32_MFMA if args.precision == "fp32_mfma" else pkg.PRECISION_FP32


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--seconds", type=float, default=60.0, help="mix length")
    ap.add_argument("--batch-chunks", type=int, default=8)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--attn-iters", type=int, default=20)
    ap.add_argument("--roofline-only", action="store_true",
                    help="only the roofline kernel loop and the copy calibration (for rocprofv3 runs)")
    ap.add_argument("--no-other-configs", action="store_true",
                    help="skip the config 2 / 4 / 5 measurements reported beside the headline")
    ap.add_argument("--profile", choices=("host", "device", "bf16"),
                    help="for rocprofv3 runs: only --warmup + --steps of one workload and one short JSON line: "
                         "host = the config-3 separation from host arrays (dmx_separate), device = the same with "
                         "mix and stems in HBM (dmx_separate_device), bf16 = the config-5 forward of 32 segments; "
                         "each followed by the 256 MiB copy that calibrates the traffic counters")
    ap.add_argument("--precision", choices=("fp32", "fp32_mfma"), default="fp32",
                    help="fp32 workloads: fp32 = the default runner precision (transformer linears on three bf16 "
                         "planes per operand, fp32-accurate); fp32_mfma = fp32 MFMA for every contraction")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs on one GPU only; multi-GPU runs are not part of it "
              "(the path would shard by chunk ranges: each GPU a contiguous run of chunks, "
              "exchanging its overlap-add halo with its neighbour)", file=sys.stderr)
        sys.exit(2)

    import torch
    pkg = load_package()
    if args.roofline_only:
        attn_ms, attn_flops = attention_roofline(pkg, torch, args.batch_chunks, args.attn_iters,
                                                 fp32_precision(pkg, args), planes_attention(args))
        mib = copy_calibration(torch)
        print(json.dumps({"kernel": "attention_x3_kernel" if planes_attention(args) else "attention_kernel",
                          "avg_ms": round(attn_ms, 4),
                          "tflops": round(attn_flops / (attn_ms * 1e-3) / 1e12, 2),
                          "flops_per_launch": attn_flops, "copy_calibration_mib": mib}))
        return
    if args.profile:
        print(json.dumps(profile_workload(pkg, torch, args)))
        return
    cfg = pkg.Config()
    weights = pkg.random_init(0, cfg)
    runner = pkg.Runner(weights, cfg, device=0, precision=fp32_precision(pkg, args))
    mix = pkg.signals.synthetic_mix(0, args.seconds)
    samples = mix.shape[1]
    audio_s = samples / cfg.samplerate
    opts = pkg.SeparateOptions(shifts=0, overlap=0.25, batch_chunks=args.batch_chunks)
    left, right = np.ascontiguousarray(mix[0]), np.ascontiguousarray(mix[1])

    # The metric: host f32 mix in, host f32 stems out, one fresh output array
    # per call as a caller of Demucs::separate gets.
    def step():
        return pkg.separate_runners([runner], left, right, cfg.samplerate, opts)

    for _ in range(args.warmup):
        step()
    runner.synchronize()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        stems = step()
    runner.synchronize()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_per_step = 1000.0 * elapsed / args.steps
    xrt = audio_s * args.steps / elapsed
    if not np.isfinite(stems).all():
        raise RuntimeError("non-finite stems")

    # The same separation with the mix and the stems resident in HBM
    # (dmx_separate_device), over the same number of steps.
    d_mix = torch.from_numpy(mix).cuda()
    d_stems = torch.empty((cfg.sources, 2, samples), device="cuda")
    c_opts = opts.to_c()
    lib = pkg._native.load()
    handles = (ctypes.c_void_p * 1)(runner.handle)

    def device_step():
        rc = lib.dmx_separate_device(handles, None, 1, None, ctypes.c_void_p(d_mix.data_ptr()), samples,
                                     cfg.samplerate, ctypes.byref(c_opts), pkg._native.PROGRESS(), None,
                                     ctypes.c_void_p(d_stems.data_ptr()))
        if rc != 0:
            raise RuntimeError(pkg._native.last_error())

    for _ in range(max(1, args.warmup)):
        device_step()
    runner.synchronize()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        device_step()
    runner.synchronize()
    torch.cuda.synchronize()
    dev_s = (time.perf_counter() - t0) / args.steps
    dev_stems = d_stems.cpu().numpy()
    dev_snr = min(10.0 * np.log10(np.sum(dev_stems[i].astype(np.float64) ** 2) /
                                  max(float(np.sum((dev_stems[i].astype(np.float64) - stems[i]) ** 2)), 1e-30))
                  for i in range(cfg.sources))
    device_resident = {"x_realtime": round(audio_s / dev_s, 2), "ms": round(1000.0 * dev_s, 2),
                       "min_stem_snr_db_vs_value_run": round(float(dev_snr), 1),
                       "note": "mix and stems resident in HBM (dmx_separate_device), mean over the same steps"}
    del d_mix, d_stems

    segment_forward = segment_forward_path(pkg, runner, mix, args.batch_chunks, stems)

    attn_ms, attn_flops = attention_roofline(pkg, torch, args.batch_chunks, args.attn_iters,
                                             fp32_precision(pkg, args), planes_attention(args))
    attn_tflops = attn_flops / (attn_ms * 1e-3) / 1e12
    traffic, traffic_source = measured_traffic()
    roofline = attention_roofline_record(args, attn_ms, attn_tflops, traffic, traffic_source)
    line = {
        "metric": "htdemucs x-realtime (audio s / wall s) on 1 MI355X; cross-attn TFLOP/s",
        "value": round(xrt, 2),
        "unit": "x-realtime",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded 60 s mix: 16 sinusoids + pink noise + decaying bursts; random-init seed-0 weights)",
        "config": {"workload": f"config 3: htdemucs separation of a {args.seconds:g} s stereo mix, 7.8 s segments, "
                               f"overlap 0.25, {args.batch_chunks} chunks per launch, shifts=0, fp32, "
                               "host f32 mix in to host f32 stems out (dmx_separate)",
                   "segment_samples": cfg.training_length, "batch_chunks": args.batch_chunks},
        "cross_attn_tflops": round(attn_tflops, 2),
        "device_resident": device_resident,
        "segment_forward": segment_forward,
        "roofline": roofline,
        "cpu_baseline": None if args.no_cpu_baseline else cpu_baseline(pkg, args.seconds, args.batch_chunks),
    }
    if not args.no_other_configs:
        del runner
        line["other_configs"] = {"config2_transformer": config2_transformer(pkg, torch),
                                 "config4_bag": config4_bag(pkg, torch),
                                 "config5_bf16": config5_bf16(pkg, torch)}
    print(json.dumps(line))


if __name__ == "__main__":
    main()
