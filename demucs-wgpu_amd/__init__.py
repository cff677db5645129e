"""MI355X-native HTDemucs v4 backend — the host-side mirror of the reference facade.

The reference exposes `Demucs::load(path, LoadOptions, Backend)`,
`separate` / `separate_with_progress` / `separate_with_options`, `StemSelection`
and the per-chunk `SegmentForward` (crates/demucs-core/src/api.rs:141-447,
crates/demucs-core/src/demucs/pipeline.rs:178-190). This package offers the
same surface over the C-ABI of include/dmx.h (libdmx.so, HIP kernels for
gfx950), with weights given as a name -> array mapping in checkpoint naming.

There is no CPU implementation here: the HIP library is the only compute path,
and a missing library or device raises instead of falling back.
"""
from __future__ import annotations

import ctypes
import enum
from dataclasses import dataclass, field
from typing import Callable, Dict, List, Mapping, Optional, Sequence

import numpy as np

from . import _native, audio, signals
from .config import Config
from .checkpoint import LoadedWeights, config_from_kwargs, load_weights, load_weights_from_bytes
from .weights import random_init, weight_shapes, xavier_transformer_init

__all__ = [
    "Backend", "Config", "Demucs", "DmxError", "LoadOptions", "LoadedWeights", "ModelVariant", "Runner",
    "SeparateOptions", "SeparationProgress", "Stem", "StemId", "StemSelection", "config_from_kwargs",
    "load_weights", "load_weights_from_bytes", "random_init", "weight_shapes", "xavier_transformer_init",
]

# dmx_status -> reference Error variant (crates/demucs-core/src/error.rs:4-55)
STATUS_NAMES = {1: "Shape", 2: "Config", 3: "MissingWeight", 4: "WeightShape", 5: "UnsupportedModel", 6: "Gpu",
                7: "Memory", 8: "Argument", 9: "Checkpoint", 10: "Io", 11: "Audio"}
# dmx_precision (include/dmx.h): fp32 results with the transformer linears on
# three bf16 planes per operand; bf16 MFMA inputs; fp32 MFMA everywhere.
PRECISION_FP32, PRECISION_BF16, PRECISION_FP32_MFMA = 0, 1, 2


class DmxError(RuntimeError):
    def __init__(self, code: int, message: str):
        self.code = code
        self.kind = STATUS_NAMES.get(code, "Unknown")
        super().__init__(f"{self.kind} error: {message}")


def _check(rc: int) -> None:
    if rc != 0:
        raise DmxError(rc, _native.last_error())


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _ptr(a: np.ndarray) -> ctypes.c_void_p:
    return ctypes.c_void_p(a.ctypes.data)


class StemId(enum.Enum):
    """`StemId` (api.rs:52-82), in the model's source order."""
    DRUMS = "drums"
    BASS = "bass"
    OTHER = "other"
    VOCALS = "vocals"

    @classmethod
    def parse(cls, name: str) -> Optional["StemId"]:
        for s in cls:
            if s.value == name:
                return s
        return None


class ModelVariant(enum.Enum):
    HTDEMUCS = "htdemucs"
    HTDEMUCS_FT = "htdemucs_ft"


@dataclass
class StemSelection:
    """`StemSelection::All` (stems=None) or `StemSelection::Some(list)`."""
    stems: Optional[List[StemId]] = None

    @classmethod
    def all(cls) -> "StemSelection":
        return cls(None)

    @classmethod
    def some(cls, stems: Sequence[StemId]) -> "StemSelection":
        return cls(list(stems))

    def wants(self, stem: StemId) -> bool:
        return self.stems is None or stem in self.stems


@dataclass
class LoadOptions:
    variant: ModelVariant = ModelVariant.HTDEMUCS
    stems: StemSelection = field(default_factory=StemSelection.all)


@dataclass(frozen=True)
class Backend:
    """`Backend` (api.rs:141-165) plus the HIP variant this package provides.

    `Backend.hip(n)` requires device n; `Backend.auto()` takes device 0 and
    raises when none opens (the host fallback is the reference's own CPU
    backend, not part of this package); `Backend.cpu()` is refused."""
    kind: str = "auto"
    device: int = 0

    @classmethod
    def auto(cls) -> "Backend":
        return cls("auto", 0)

    @classmethod
    def cpu(cls) -> "Backend":
        return cls("cpu", 0)

    @classmethod
    def hip(cls, device: int = 0) -> "Backend":
        return cls("hip", device)

    def tag(self) -> str:
        return "hip" if self.kind == "hip" else self.kind


@dataclass
class SeparateOptions:
    """`SeparateOptions` (pipeline.rs:16-38) plus the chunk group size (`DEMUCS_BATCH`)."""
    shifts: int = 1
    overlap: float = 0.25
    transition_power: float = 1.0
    segment: Optional[float] = None
    batch_chunks: int = 1

    def to_c(self) -> _native.CSeparateOptions:
        return _native.CSeparateOptions(self.shifts, self.overlap, self.transition_power,
                                        0.0 if self.segment is None else float(self.segment), self.batch_chunks)


@dataclass(frozen=True)
class SeparationProgress:
    """`SeparationProgress` (api.rs:198-217)."""
    done: int
    total: int

    def fraction(self) -> float:
        if self.total == 0:
            return 1.0
        return min(max(self.done / self.total, 0.0), 1.0)

    def percent(self) -> int:
        return int(self.fraction() * 100.0)


@dataclass
class Stem:
    id: StemId
    left: np.ndarray
    right: np.ndarray


class Runner:
    """One network on one device: the `GpuHtdemucsRunner` replacement
    (crates/demucs-core/src/gpu/htdemucs.rs:2335-2400)."""

    def __init__(self, weights: Mapping[str, np.ndarray], config: Optional[Config] = None, device: int = 0,
                 precision: int = PRECISION_FP32):
        self.lib = _native.load()
        self.config = config or Config()
        self._arrays = [(_f32(v), k) for k, v in weights.items()]
        entries = (_native.CTensor * len(self._arrays))()
        self._names = []
        for i, (arr, name) in enumerate(self._arrays):
            bname = name.encode()
            self._names.append(bname)
            entries[i].name = bname
            entries[i].data = arr.ctypes.data_as(_native.c_float_p)
            entries[i].ndim = arr.ndim
            for d in range(arr.ndim):
                entries[i].shape[d] = arr.shape[d]
        self._cfg = self.config.to_c()
        handle = ctypes.c_void_p()
        _check(self.lib.dmx_runner_create(entries, len(self._arrays), ctypes.byref(self._cfg), device, precision,
                                          ctypes.byref(handle)))
        self.handle = handle
        self._arrays = None  # uploaded; the runner keeps no host reference
        self._trace_cbs = None

    def close(self) -> None:
        if getattr(self, "handle", None):
            self.lib.dmx_runner_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def backend_tag(self) -> str:
        return self.lib.dmx_runner_backend_tag(self.handle).decode()

    @property
    def stream(self) -> int:
        return self.lib.dmx_runner_stream(self.handle) or 0

    def synchronize(self) -> None:
        _check(self.lib.dmx_synchronize(self.handle))

    # ---- SegmentForward ----
    def forward(self, mix: np.ndarray) -> np.ndarray:
        """`Htdemucs::forward`: (batch, 2, length) -> (batch, sources, 2, length)."""
        mix = _f32(mix)
        b, c, n = mix.shape
        out = np.empty((b, self.config.sources, c, n), dtype=np.float32)
        _check(self.lib.dmx_forward(self.handle, _ptr(mix), b, c, n, _ptr(out)))
        return out

    def start(self, mix: np.ndarray):
        mix = _f32(mix)
        b, c, n = mix.shape
        pending = ctypes.c_void_p()
        _check(self.lib.dmx_forward_start(self.handle, _ptr(mix), b, c, n, ctypes.byref(pending)))
        return (pending, (b, self.config.sources, c, n))

    def collect(self, pending) -> np.ndarray:
        handle, shape = pending
        out = np.empty(shape, dtype=np.float32)
        _check(self.lib.dmx_forward_collect(self.handle, handle, _ptr(out)))
        return out

    def forward_device(self, d_mix_ptr: int, batch: int, channels: int, length: int, d_out_ptr: int) -> None:
        _check(self.lib.dmx_forward_device(self.handle, ctypes.c_void_p(d_mix_ptr), batch, channels, length,
                                           ctypes.c_void_p(d_out_ptr)))

    def crosstransformer_device(self, d_spec: int, d_time: int, batch: int, freqs: int, frames: int, time_len: int,
                                d_spec_out: int, d_time_out: int) -> None:
        _check(self.lib.dmx_crosstransformer_device(self.handle, ctypes.c_void_p(d_spec), ctypes.c_void_p(d_time),
                                                    batch, freqs, frames, time_len, ctypes.c_void_p(d_spec_out),
                                                    ctypes.c_void_p(d_time_out)))

    def set_trace(self, wants: Optional[Callable[[str], bool]], record: Optional[Callable[[str, np.ndarray], None]]):
        """TraceSink (host.rs:117-125); pass None, None to clear."""
        if record is None:
            self._trace_cbs = None
            _check(self.lib.dmx_set_trace(self.handle, _native.TRACE_WANTS(), _native.TRACE_RECORD(), None))
            return

        def _wants(name, _user):
            return 1 if (wants is None or wants(name.decode())) else 0

        def _record(name, shape, ndim, data, _user):
            dims = tuple(shape[i] for i in range(ndim))
            arr = np.ctypeslib.as_array(data, shape=(int(np.prod(dims)),)).copy().reshape(dims)
            record(name.decode(), arr)

        self._trace_cbs = (_native.TRACE_WANTS(_wants), _native.TRACE_RECORD(_record))
        _check(self.lib.dmx_set_trace(self.handle, self._trace_cbs[0], self._trace_cbs[1], None))


def separate_runners(runners: Sequence[Runner], left: np.ndarray, right: np.ndarray, sample_rate: int,
                     options: SeparateOptions, bag_weights: Optional[np.ndarray] = None,
                     wanted: Optional[Sequence[bool]] = None,
                     on_progress: Optional[Callable[[SeparationProgress], None]] = None) -> np.ndarray:
    """dmx_separate: (sources, 2, samples) stems, unwanted rows left at zero."""
    lib = _native.load()
    left, right = _f32(left), _f32(right)
    if left.shape != right.shape:
        raise DmxError(1, f"left/right lengths differ ({left.shape[0]} vs {right.shape[0]})")
    sources = runners[0].config.sources
    out = np.zeros((sources, 2, left.shape[0]), dtype=np.float32)
    handles = (ctypes.c_void_p * len(runners))(*[r.handle for r in runners])
    w = None if bag_weights is None else _f32(bag_weights).reshape(len(runners), sources)
    mask = None if wanted is None else np.array([1 if x else 0 for x in wanted], dtype=np.uint8)
    opts = options.to_c()
    cb = _native.PROGRESS(lambda d, t, _u: on_progress(SeparationProgress(d, t))) if on_progress else _native.PROGRESS()
    _check(lib.dmx_separate(handles, None if w is None else _ptr(w), len(runners), None if mask is None else _ptr(mask),
                            _ptr(left), _ptr(right), left.shape[0], sample_rate, ctypes.byref(opts), cb, None,
                            _ptr(out)))
    return out


def separate_emit_runners(runners: Sequence[Runner], left: np.ndarray, right: np.ndarray, sample_rate: int,
                          options: SeparateOptions, on_frames: Callable[[int, np.ndarray], None],
                          bag_weights: Optional[np.ndarray] = None, wanted: Optional[Sequence[bool]] = None,
                          on_progress: Optional[Callable[[SeparationProgress], None]] = None) -> None:
    """dmx_separate_emit: `on_frames(start, stems)` receives each finished
    region in order as (sources, 2, frames) float32 (rows of unwanted stems
    are zero), while later chunk groups still compute. An exception raised by
    `on_frames` stops the separation and propagates."""
    lib = _native.load()
    left, right = _f32(left), _f32(right)
    if left.shape != right.shape:
        raise DmxError(1, f"left/right lengths differ ({left.shape[0]} vs {right.shape[0]})")
    sources = runners[0].config.sources
    handles = (ctypes.c_void_p * len(runners))(*[r.handle for r in runners])
    w = None if bag_weights is None else _f32(bag_weights).reshape(len(runners), sources)
    mask = None if wanted is None else np.array([1 if x else 0 for x in wanted], dtype=np.uint8)
    opts = options.to_c()
    failure = []

    def _emit(start, frames, rows, _user):
        try:
            block = np.zeros((sources, 2, frames), dtype=np.float32)
            for r in range(2 * sources):
                if rows[r]:
                    block[r // 2, r % 2] = np.ctypeslib.as_array(rows[r], shape=(frames,))
            on_frames(int(start), block)
            return 0
        except BaseException as exc:  # handed back after the C call returns
            failure.append(exc)
            return 1

    emit_cb = _native.EMIT(_emit)
    cb = _native.PROGRESS(lambda d, t, _u: on_progress(SeparationProgress(d, t))) if on_progress else _native.PROGRESS()
    rc = lib.dmx_separate_emit(handles, None if w is None else _ptr(w), len(runners),
                               None if mask is None else _ptr(mask), _ptr(left), _ptr(right), left.shape[0],
                               sample_rate, ctypes.byref(opts), cb, None, emit_cb, None)
    if failure:
        raise failure[0]
    _check(rc)


class Demucs:
    """`Demucs` (api.rs:374-447): one network or the fine-tuned bag."""

    def __init__(self, runners: List[Runner], bag_weights: Optional[np.ndarray], opts: LoadOptions):
        self.runners = runners
        self.bag_weights = bag_weights
        self.opts = opts

    @classmethod
    def load(cls, weights, opts: Optional[LoadOptions] = None, backend: Optional[Backend] = None,
             config: Optional[Config] = None, bag_weights: Optional[np.ndarray] = None) -> "Demucs":
        """`weights` is one network or a list of them for the bag (with
        `bag_weights` (networks x sources), identity by default). A network is
        a name -> array mapping, a `LoadedWeights`, or a checkpoint path
        (`load_weights`: torch zip or safetensors); the config of a loaded
        checkpoint is used unless `config` is given."""
        opts = opts or LoadOptions()
        backend = backend or Backend.auto()
        if backend.kind == "cpu":
            raise DmxError(5, "the CPU backend is the reference's own host path; this package provides Backend.hip")
        nets = weights if isinstance(weights, (list, tuple)) else [weights]
        runners = []
        for w in nets:
            if isinstance(w, (str, bytes)) or hasattr(w, "__fspath__"):
                w = load_weights(w)
            if isinstance(w, LoadedWeights):
                runners.append(Runner(w.tensors, config or w.config, backend.device))
            else:
                runners.append(Runner(w, config, backend.device))
        if len(runners) > 1 and bag_weights is None:
            bag_weights = np.eye(len(runners), runners[0].config.sources, dtype=np.float32)
        return cls(runners, bag_weights, opts)

    @property
    def backend_tag(self) -> str:
        return self.runners[0].backend_tag

    @property
    def sources(self) -> List[str]:
        return list(Config.SOURCES[: self.runners[0].config.sources])

    @property
    def sample_rate(self) -> int:
        return self.runners[0].config.samplerate

    def forward_segment(self, mix: np.ndarray) -> np.ndarray:
        if len(self.runners) != 1:
            raise DmxError(1, "forward_segment is per network")
        return self.runners[0].forward(mix)

    def separate(self, left, right, sample_rate: int) -> List[Stem]:
        return self.separate_with_options(left, right, sample_rate, SeparateOptions())

    def separate_with_progress(self, left, right, sample_rate: int,
                               on_progress: Callable[[SeparationProgress], None]) -> List[Stem]:
        return self.separate_with_options(left, right, sample_rate, SeparateOptions(), on_progress)

    def separate_with_options(self, left, right, sample_rate: int, options: SeparateOptions,
                              on_progress: Optional[Callable[[SeparationProgress], None]] = None) -> List[Stem]:
        ids = [StemId.parse(n) for n in self.sources]
        wanted = [self.opts.stems.wants(i) for i in ids]
        out = separate_runners(self.runners, left, right, sample_rate, options, self.bag_weights, wanted, on_progress)
        return [Stem(i, out[k, 0].copy(), out[k, 1].copy()) for k, i in enumerate(ids) if wanted[k]]

    def separate_streaming(self, left, right, sample_rate: int, options: SeparateOptions,
                           on_frames: Callable[[int, np.ndarray], None],
                           on_progress: Optional[Callable[[SeparationProgress], None]] = None) -> None:
        """`separate_streaming` (api.rs:617-654) a region at a time: each
        finished region of denormalised stems goes to `on_frames(start,
        stems)` in order, stems (sources, 2, frames) with unwanted rows zero,
        while later chunk groups still compute."""
        ids = [StemId.parse(n) for n in self.sources]
        wanted = [self.opts.stems.wants(i) for i in ids]
        separate_emit_runners(self.runners, left, right, sample_rate, options, on_frames, self.bag_weights, wanted,
                              on_progress)

    def _read_mix(self, path) -> np.ndarray:
        from .audio import read_audio
        a = read_audio(path).ensure_channels(2)
        if a.sample_rate != self.sample_rate:
            raise DmxError(1, f"{path} is at {a.sample_rate} Hz but the model wants {self.sample_rate} Hz")
        return a.data

    def separate_file(self, path, on_progress: Optional[Callable[[SeparationProgress], None]] = None,
                      options: Optional[SeparateOptions] = None) -> List[Stem]:
        """`separate_file` (api.rs:786-818): a WAV file (mono duplicated to
        stereo) at the model's rate; every requested stem."""
        mix = self._read_mix(path)
        return self.separate_with_options(mix[0], mix[1], self.sample_rate, options or SeparateOptions(), on_progress)

    def separate_streaming_file(self, path, options: SeparateOptions, on_frames: Callable[[int, np.ndarray], None],
                                on_progress: Optional[Callable[[SeparationProgress], None]] = None) -> None:
        """`separate_streaming_file` (api.rs:656-695): separate_streaming of a WAV file."""
        mix = self._read_mix(path)
        self.separate_streaming(mix[0], mix[1], self.sample_rate, options, on_frames, on_progress)
