"""`demucs` command line over the HIP backend: separate, info, compare, bench.

Mirrors the reference CLI (crates/demucs-cli/src/main.rs): the same
subcommands, flags and messages for the paths this backend provides. Run it
as `python demucs-wgpu_amd <command> ...` (the package directory's
__main__.py) or call `main(argv)`.

Models (`--model`): a checkpoint file (.th or .safetensors), a directory
holding htdemucs_ft.yaml and its networks' .safetensors (the fine-tuned bag),
or `random:SEED[,SEED...]` for this build's seeded random-init weights (one
network, or an identity bag of several), since no published checkpoint ships
with it. Devices (`--device`): `auto`, `gpu`, `hip` or `hip:N`; `cpu` is the
reference's own host backend and is refused.
"""
from __future__ import annotations

import argparse
import os
import sys
import time
from pathlib import Path
from typing import List, Optional, Sequence, Tuple

import numpy as np


def _pkg():
    return sys.modules[__name__.rsplit(".", 1)[0]]


class CliError(RuntimeError):
    pass


def parse_device(spec: str):
    """`--device` (main.rs:66-88): auto, gpu, hip or hip:N select a HIP
    device; cpu names the reference's host path, which this package does
    not ship."""
    pkg = _pkg()
    s = (spec or "auto").strip().lower()
    if s in ("", "auto", "gpu", "hip"):
        return pkg.Backend.hip(0) if s != "auto" else pkg.Backend.auto()
    if s.startswith("hip:"):
        try:
            return pkg.Backend.hip(int(s[4:]))
        except ValueError:
            raise CliError(f"--device {spec!r}: expected hip:<index>")
    if s == "cpu":
        raise CliError("--device cpu is the reference's host backend; this build runs on HIP devices only "
                       "(use auto, gpu or hip:<index>)")
    raise CliError(f"--device {spec!r}: expected auto, gpu, hip or hip:<index>")


def _bag_dir(path: Path) -> Tuple[List[Path], np.ndarray]:
    """htdemucs_ft.yaml of a snapshot directory: `models` (network names, one
    <name>.safetensors each) and `weights` (one row of per-source weights per
    network), as api.rs:1047-1081 reads it."""
    import yaml
    spec = yaml.safe_load((path / "htdemucs_ft.yaml").read_text())
    if not isinstance(spec, dict) or "models" not in spec or "weights" not in spec:
        raise CliError(f"{path / 'htdemucs_ft.yaml'}: needs `models` and `weights`")
    names = [str(n) for n in spec["models"]]
    weights = np.asarray(spec["weights"], dtype=np.float32)
    if weights.ndim != 2 or weights.shape[0] != len(names):
        raise CliError(f"htdemucs_ft.yaml lists {len(names)} networks but {weights.shape[0]} weight rows")
    return [path / f"{n}.safetensors" for n in names], weights


def load_model(spec: str, backend, stems=None, precision: int = 0, segment: Optional[float] = None):
    """`--model` -> (Demucs, seconds to load, parameter count per network)."""
    pkg = _pkg()
    opts = pkg.LoadOptions(stems=stems or pkg.StemSelection.all())
    started = time.perf_counter()
    if backend.kind == "cpu":
        raise CliError("the CPU backend is the reference's own")
    nets, bag = [], None
    cfg = pkg.Config()
    if spec.startswith("random:"):
        seeds = [int(x) for x in spec[len("random:"):].split(",") if x.strip()]
        if not seeds:
            raise CliError("--model random:SEED[,SEED...]")
        nets = [(pkg.random_init(sd, cfg), cfg) for sd in seeds]
        if len(seeds) > 1:
            bag = np.eye(len(seeds), cfg.sources, dtype=np.float32)
    else:
        path = Path(spec)
        if path.is_dir():
            if not (path / "htdemucs_ft.yaml").exists():
                raise CliError(f"{path} is a directory but has no htdemucs_ft.yaml")
            files, bag = _bag_dir(path)
            opts.variant = pkg.ModelVariant.HTDEMUCS_FT
        elif path.exists():
            files = [path]
        else:
            raise CliError(f"{spec}: no such checkpoint (a .th/.safetensors file, an htdemucs_ft directory, "
                           "or random:SEED)")
        for f in files:
            loaded = pkg.load_weights(f)
            nets.append((loaded.tensors, loaded.config))
    if segment is not None:
        for _, c in nets:
            c.segment = float(segment)
    runners = [pkg.Runner(w, c, backend.device, precision) for w, c in nets]
    model = pkg.Demucs(runners, bag, opts)
    count = pkg.weights.parameter_count(nets[0][0])
    return model, time.perf_counter() - started, count


def report(audio_seconds: float, elapsed: float, load_seconds: float, timings: bool, samplerate: int,
           segment: float) -> None:
    """The summary line of main.rs:563-587."""
    print(f"separation {elapsed:.2f}s for {audio_seconds:.3f}s -> RTFx {audio_seconds / elapsed:.2f}x | "
          f"+ {load_seconds:.2f}s load = end-to-end RTFx {audio_seconds / (elapsed + load_seconds):.2f}x")
    if timings:
        seg_len = int(samplerate * segment)
        stride = int(0.75 * seg_len)
        chunks = audio_seconds * samplerate / stride
        print(f"per chunk: {elapsed / chunks * 1000.0:.0f} ms of model input, "
              f"{segment / (elapsed / chunks):.1f}x raw ({chunks:.0f} chunks)")


def separate(args) -> int:
    """`separate` (main.rs:313-556): one float WAV per requested stem, written
    region by region as the separation finishes them."""
    pkg = _pkg()
    backend = parse_device(args.device)
    names = list(pkg.Config.SOURCES)
    requested = args.stem or args.two_stems
    if requested is not None and requested not in names:
        raise CliError(f"--stem/--two-stems must be one of {names}, got {requested!r}")
    method = args.other_method if args.two_stems else "none"
    # Only a request that writes just the named stem prunes the bag to the
    # network that produces it (main.rs:332-343).
    prune = args.stem is not None or (args.two_stems is not None and method == "none")
    stems = pkg.StemSelection.some([pkg.StemId.parse(requested)]) if (requested and prune) else None
    precision = pkg.PRECISION_BF16 if args.precision == "bf16" else pkg.PRECISION_FP32
    model, load_seconds, _ = load_model(args.model, backend, stems, precision, args.segment)
    audio = pkg.audio.read_audio(args.input).ensure_channels(2)
    if audio.sample_rate != model.sample_rate:
        raise CliError(f"{args.input} is at {audio.sample_rate} Hz but the model wants {model.sample_rate} Hz")
    mix = audio.data
    selected = [(names.index(requested), requested)] if requested else list(enumerate(names))
    companion = None
    if args.two_stems and method != "none":
        companion = (("no_" if method == "add" else "minus_") + requested, method, names.index(requested))
    out = Path(args.output)
    single_file = companion is None and out.suffix != "" and len(selected) == 1
    if not single_file:
        out.mkdir(parents=True, exist_ok=True)
    path_for = (lambda name: out) if single_file else (lambda name: out / f"{name}.wav")
    writers = [(i, n, pkg.audio.FloatWavWriter(path_for(n), model.sample_rate, 2)) for i, n in selected]
    comp_writer = pkg.audio.FloatWavWriter(path_for(companion[0]), model.sample_rate, 2) if companion else None
    peaks = {n: 0.0 for _, n, _ in writers}
    if companion:
        peaks[companion[0]] = 0.0

    def on_frames(start: int, block: np.ndarray) -> None:
        n = block.shape[-1]
        for i, name, w in writers:
            w.write_planar(block[i])
            peaks[name] = max(peaks[name], float(np.abs(block[i]).max(initial=0.0)))
        if comp_writer is not None:
            _, how, idx = companion
            if how == "add":
                rows = block.sum(axis=0) - block[idx]
            else:
                rows = mix[:, start:start + n] - block[idx]
            comp_writer.write_planar(rows)
            peaks[companion[0]] = max(peaks[companion[0]], float(np.abs(rows).max(initial=0.0)))

    options = pkg.SeparateOptions(shifts=args.shifts, overlap=args.overlap, segment=args.segment,
                                  batch_chunks=args.batch_chunks)
    started = time.perf_counter()
    model.separate_streaming(mix[0], mix[1], model.sample_rate, options, on_frames)
    elapsed = time.perf_counter() - started
    written = []
    for _, name, w in writers:
        w.finish()
        written.append(f"{path_for(name)} (peak {peaks[name]:.4f})")
    if comp_writer is not None:
        comp_writer.finish()
        written.append(f"{path_for(companion[0])} (peak {peaks[companion[0]]:.4f})")
    seg = args.segment if args.segment else model.runners[0].config.segment
    report(mix.shape[1] / model.sample_rate, elapsed, load_seconds, args.timings, model.sample_rate, seg)
    print("wrote " + ", ".join(written))
    return 0


def layer_table(cfg) -> List[str]:
    """The architecture `info` prints (main.rs:239-275), derived from the config."""
    rows = []
    chin, freqs = cfg.audio_channels * (2 if cfg.cac else 1), cfg.nfft // 2
    tchin = cfg.audio_channels
    enc, tenc = [], []
    for i in range(cfg.depth):
        chout = cfg.channels * cfg.growth ** i
        enc.append(f"  encoder.{i} {freqs:>5} bins, {chin:>3} -> {chout:>3} channels, "
                   f"k={cfg.kernel_size} s={cfg.stride} p={cfg.kernel_size // 4}")
        tenc.append(f"  tencoder.{i} {tchin:>3} -> {chout:>3} channels, "
                    f"k={cfg.kernel_size} s={cfg.stride} p={cfg.kernel_size // 4}")
        chin, tchin, freqs = chout, chout, freqs // cfg.stride
    rows.append("frequency branch:")
    rows += enc
    rows.append(f"  bottleneck: {freqs} bins, {chin} channels")
    rows.append("waveform branch:")
    rows += tenc
    rows.append("decoder (execution order):")
    for i in range(cfg.depth):
        level = cfg.depth - 1 - i
        cin = cfg.channels * cfg.growth ** level
        cout = cfg.channels * cfg.growth ** (level - 1) if level > 0 else cfg.sources * cfg.audio_channels * \
            (2 if cfg.cac else 1)
        rows.append(f"  decoder.{i} {cin:>3} -> {cout:>3} channels")
    return rows


def info(args) -> int:
    """`info` (main.rs:224-277): parameter count, config and layer table."""
    pkg = _pkg()
    started = time.perf_counter()
    if args.model.startswith("random:"):
        cfg = pkg.Config()
        weights = pkg.random_init(int(args.model.split(":", 1)[1].split(",")[0]), cfg)
    else:
        loaded = pkg.load_weights(args.model)
        weights, cfg = loaded.tensors, loaded.config
    seconds = time.perf_counter() - started
    print(f"loaded in {seconds:.2f}s | {pkg.weights.parameter_count(weights)} parameters | {cfg.sources} sources "
          f"{list(pkg.Config.SOURCES[:cfg.sources])} | segment {cfg.segment:.3f}s")
    print(f"nfft {cfg.nfft} hop {cfg.hop_length} depth {cfg.depth} channels {cfg.channels} transformer "
          f"{cfg.bottom_channels} layers {cfg.t_layers} heads {cfg.t_heads}")
    for row in layer_table(cfg):
        print(row)
    return 0


def compare(args) -> int:
    """`compare` (main.rs:282-301): the fixtures' SNR between two WAVs."""
    pkg = _pkg()
    a = pkg.audio.read_audio(args.reference)
    b = pkg.audio.read_audio(args.other)
    if a.data.shape != b.data.shape:
        raise CliError(f"shape mismatch: {a.channels}x{a.samples} vs {b.channels}x{b.samples}")
    r = pkg.audio.compare(a.data, b.data)
    print(f"{args.reference} vs {args.other}: {r.snr_db():.2f} dB SNR (max abs {r.max_abs:.3e}, "
          f"reference peak {r.reference_max_abs:.6f})")
    return 0


def bench_mix(channels: int, length: int) -> np.ndarray:
    """The bench input of main.rs:1130-1135: an LCG's uniform values in
    [-0.1, 0.1), channel-major."""
    out = np.empty(channels * length, dtype=np.float32)
    state = 12345
    for i in range(out.size):
        state = (state * 1664525 + 1013904223) & 0xFFFFFFFF
        out[i] = ((state >> 8) / 8388608.0 - 1.0) * 0.1
    return out.reshape(1, channels, length)


def bench(args) -> int:
    """`bench` (main.rs:1126-1190): one segment's forward on the device,
    averaged over `repeats` after a warm-up, with the readback included."""
    pkg = _pkg()
    backend = parse_device(args.device)
    model, load_seconds, count = load_model(args.model, backend)
    print(f"load {load_seconds:.2f}s, {count} parameters")
    runner = model.runners[0]
    length = runner.config.training_length
    mix = bench_mix(runner.config.audio_channels, length)
    runner.forward(mix)
    started = time.perf_counter()
    for _ in range(args.repeats):
        runner.forward(mix)
    elapsed = (time.perf_counter() - started) / args.repeats
    seconds = length / runner.config.samplerate
    print(f"chunk forward {elapsed * 1000.0:.1f} ms for {seconds:.3f}s of audio -> {seconds / elapsed:.2f}x raw "
          f"({seconds * runner.config.audio_channels * 4.0 / elapsed / 1e9:.1f} GB/s of input audio)")
    return 0


def build_parser() -> argparse.ArgumentParser:
    p = argparse.ArgumentParser(prog="demucs", description="HTDemucs separation (MI355X HIP backend)")
    sub = p.add_subparsers(dest="command", required=True)
    s = sub.add_parser("separate", help="Separate a track and write one WAV per stem.")
    s.add_argument("input")
    s.add_argument("-o", "--output", required=True, help="output directory (one <stem>.wav each) or a .wav path")
    s.add_argument("-m", "--model", default="random:0", help="checkpoint, htdemucs_ft directory or random:SEED")
    g = s.add_mutually_exclusive_group()
    g.add_argument("--stem", help="only write this stem")
    g.add_argument("--two-stems", help="write STEM and no_STEM (or minus_STEM)")
    s.add_argument("--other-method", choices=("add", "minus", "none"), default="add")
    s.add_argument("--shifts", type=int, default=1)
    s.add_argument("--overlap", type=float, default=0.25)
    s.add_argument("--segment", type=float, default=None)
    s.add_argument("--device", default="auto")
    s.add_argument("--batch-chunks", type=int, default=8, help="chunks per forward launch (DEMUCS_BATCH)")
    s.add_argument("--precision", choices=("fp32", "bf16"), default="fp32")
    s.add_argument("--timings", action="store_true")
    s.set_defaults(func=separate)
    i = sub.add_parser("info", help="Print the model's parameter count, config and layer table.")
    i.add_argument("-m", "--model", default="random:0")
    i.set_defaults(func=info)
    c = sub.add_parser("compare", help="Compare two WAV files and report the SNR between them.")
    c.add_argument("reference")
    c.add_argument("other")
    c.set_defaults(func=compare)
    b = sub.add_parser("bench", help="Run the network on one segment and print the timings.")
    b.add_argument("-m", "--model", default="random:0")
    b.add_argument("-r", "--repeats", type=int, default=3)
    b.add_argument("--device", default="auto")
    b.set_defaults(func=bench)
    return p


def main(argv: Optional[Sequence[str]] = None) -> int:
    args = build_parser().parse_args(argv)
    pkg = _pkg()
    from .checkpoint import CheckpointError
    try:
        return args.func(args)
    except (CliError, pkg.DmxError, CheckpointError) as e:
        print(f"demucs: {e}", file=sys.stderr)
        return 1
