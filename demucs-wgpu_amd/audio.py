"""Audio files and the stem comparison, over include/dmx_audio.h.

Mirrors crates/demucs-core/src/audio.rs (read_audio, probe_audio, write_wav,
write_wav_f32, FloatWavWriter, Subtype, Audio::ensure_channels) and
crates/demucs-core/src/fixtures.rs (compare, Comparison) for WAV files. The
decoding and encoding run in libdmx.so; samples are float32, channel-major
(channels, frames), as the reference's Audio holds them.
"""
from __future__ import annotations

import ctypes
import enum
import os
from dataclasses import dataclass

import numpy as np

from . import _native


def _check(rc: int) -> None:
    if rc != 0:
        from . import DmxError
        raise DmxError(rc, _native.last_error())


def _path(p) -> bytes:
    return os.fsencode(os.fspath(p))


@dataclass
class AudioInfo:
    """AudioInfo (audio.rs:60-66): header facts without the samples."""
    sample_rate: int
    channels: int
    frames: int


@dataclass
class Audio:
    """Audio (audio.rs:13-57): `data` is (channels, frames) float32."""
    sample_rate: int
    data: np.ndarray

    @property
    def channels(self) -> int:
        return self.data.shape[0]

    @property
    def samples(self) -> int:
        return self.data.shape[1]

    def channel(self, index: int) -> np.ndarray:
        return self.data[index]

    def ensure_channels(self, wanted: int) -> "Audio":
        """Mono is duplicated when two channels are wanted (inference.py's
        expansion, audio.rs:37-57); any other mismatch is an Audio error."""
        if self.channels == wanted:
            return self
        if self.channels == 1 and wanted == 2:
            return Audio(self.sample_rate, np.concatenate([self.data, self.data], axis=0))
        from . import DmxError
        raise DmxError(11, f"cannot convert {self.channels} channels to {wanted}")


class Subtype(enum.IntEnum):
    """sf.write subtypes a WAV can be written in (audio.rs:366-411)."""
    PCM_16 = 0
    PCM_24 = 1
    FLOAT = 2

    @classmethod
    def parse(cls, name: str) -> "Subtype":
        return cls[name]


def probe_audio(path) -> AudioInfo:
    """probe_audio (audio.rs:69-97): rate, channels and frames of a WAV."""
    info = _native.CAudioInfo()
    _check(_native.load().dmx_audio_probe(_path(path), ctypes.byref(info)))
    return AudioInfo(info.sample_rate, info.channels, info.frames)


def read_audio(path) -> Audio:
    """read_audio (audio.rs:100-112) for WAV: PCM 16/24/32 bits (scaled by
    2^-(bits-1)) or IEEE float 32/64 bits."""
    lib = _native.load()
    head = probe_audio(path)
    data = np.empty((head.channels, head.frames), dtype=np.float32)
    info = _native.CAudioInfo()
    _check(lib.dmx_audio_read(_path(path), ctypes.c_void_p(data.ctypes.data), data.size, ctypes.byref(info)))
    if (info.channels, info.frames) != (head.channels, head.frames):
        from . import DmxError
        raise DmxError(11, f"{path}: changed while it was read")
    return Audio(info.sample_rate, data)


def write_wav(path, subtype: Subtype, sample_rate: int, data) -> None:
    """write_wav (audio.rs:464-545): `data` (channels, frames), written
    interleaved in `subtype`."""
    a = np.ascontiguousarray(data, dtype=np.float32)
    if a.ndim == 1:
        a = a[None]
    _check(_native.load().dmx_wav_write(_path(path), int(subtype), int(sample_rate), a.shape[0],
                                        ctypes.c_void_p(a.ctypes.data), a.shape[1]))


def write_wav_f32(path, sample_rate: int, data) -> None:
    """write_wav_f32 (audio.rs:547-555): an IEEE float WAV."""
    write_wav(path, Subtype.FLOAT, sample_rate, data)


class FloatWavWriter:
    """FloatWavWriter (audio.rs:556-669): an IEEE float WAV written frame by
    frame; finish() patches its sizes. Usable as a context manager."""

    def __init__(self, path, sample_rate: int, channels: int):
        self._lib = _native.load()
        self._h = ctypes.c_void_p()
        _check(self._lib.dmx_wav_writer_create(_path(path), int(sample_rate), int(channels), ctypes.byref(self._h)))
        self.sample_rate = int(sample_rate)
        self.channels = int(channels)

    @classmethod
    def create(cls, path, sample_rate: int, channels: int) -> "FloatWavWriter":
        return cls(path, sample_rate, channels)

    def _live(self):
        if not self._h:
            from . import DmxError
            raise DmxError(8, "the writer is finished")
        return self._h

    def write_frame(self, frame) -> None:
        self.write_interleaved(frame)

    def write_interleaved(self, interleaved) -> None:
        a = np.ascontiguousarray(interleaved, dtype=np.float32).reshape(-1)
        if a.size % self.channels:
            from . import DmxError
            raise DmxError(11, f"{a.size} samples do not divide into {self.channels} channels")
        _check(self._lib.dmx_wav_writer_write(self._live(), ctypes.c_void_p(a.ctypes.data), a.size // self.channels))

    def write_planar(self, rows) -> None:
        """Appends (channels, n) samples, one row per channel."""
        a = np.ascontiguousarray(rows, dtype=np.float32)
        if a.ndim != 2 or a.shape[0] != self.channels:
            from . import DmxError
            raise DmxError(11, f"expected ({self.channels}, frames) rows, got {a.shape}")
        _check(self._lib.dmx_wav_writer_write_planar(self._live(), ctypes.c_void_p(a.ctypes.data), a.shape[1],
                                                     a.shape[1]))

    def frames_written(self) -> int:
        return int(self._lib.dmx_wav_writer_frames(self._h)) if self._h else 0

    def finish(self) -> None:
        h, self._h = self._live(), ctypes.c_void_p()
        _check(self._lib.dmx_wav_writer_finish(h))

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        if self._h:
            self.finish()

    def __del__(self):
        if getattr(self, "_h", None):
            self._lib.dmx_wav_writer_finish(self._h)


@dataclass
class Comparison:
    """Comparison (fixtures.rs:98-150)."""
    elements: int
    max_abs: float
    max_abs_index: int
    max_rel: float
    mean_abs: float
    reference_max_abs: float
    reference_rms: float
    _rms_relative_error: float
    _snr_db: float

    def normalized_error(self) -> float:
        return self.max_abs / self.reference_max_abs if self.reference_max_abs > 0 else self.max_abs

    def rms_relative_error(self) -> float:
        return self._rms_relative_error

    def snr_db(self) -> float:
        return self._snr_db


def compare(expected, actual) -> Comparison:
    """compare (fixtures.rs:152-189) of two flat float32 buffers."""
    e = np.ascontiguousarray(expected, dtype=np.float32).reshape(-1)
    a = np.ascontiguousarray(actual, dtype=np.float32).reshape(-1)
    if e.size != a.size:
        from . import DmxError
        raise DmxError(1, f"cannot compare {e.size} elements against {a.size}")
    r = _native.CComparison()
    _check(_native.load().dmx_compare(ctypes.c_void_p(e.ctypes.data), ctypes.c_void_p(a.ctypes.data), e.size,
                                      ctypes.byref(r)))
    return Comparison(r.elements, r.max_abs, r.max_abs_index, r.max_rel, r.mean_abs, r.reference_max_abs,
                      r.reference_rms, r.rms_relative_error, r.snr_db)
