"""HtdemucsConfig mirror (crates/demucs-core/src/demucs/config.rs:18-71) and
its C layout (``dmx_config`` of include/dmx.h)."""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, fields


class CConfig(ctypes.Structure):
    _fields_ = [
        ("sources", ctypes.c_int32),
        ("audio_channels", ctypes.c_int32),
        ("samplerate", ctypes.c_int32),
        ("segment", ctypes.c_double),
        ("channels", ctypes.c_int32),
        ("growth", ctypes.c_int32),
        ("nfft", ctypes.c_int32),
        ("depth", ctypes.c_int32),
        ("stride", ctypes.c_int32),
        ("kernel_size", ctypes.c_int32),
        ("context", ctypes.c_int32),
        ("freq_emb", ctypes.c_double),
        ("emb_scale", ctypes.c_double),
        ("cac", ctypes.c_int32),
        ("bottom_channels", ctypes.c_int32),
        ("t_layers", ctypes.c_int32),
        ("t_heads", ctypes.c_int32),
        ("t_hidden_scale", ctypes.c_double),
        ("t_max_period", ctypes.c_double),
        ("t_weight_pos_embed", ctypes.c_double),
    ]


@dataclass
class Config:
    """Defaults of `HtdemucsConfig::default` (the htdemucs / htdemucs_ft architecture)."""

    sources: int = 4
    audio_channels: int = 2
    samplerate: int = 44100
    segment: float = 39.0 / 5.0
    channels: int = 48
    growth: int = 2
    nfft: int = 4096
    depth: int = 4
    stride: int = 4
    kernel_size: int = 8
    context: int = 1
    freq_emb: float = 0.2
    emb_scale: float = 10.0
    cac: int = 1
    bottom_channels: int = 512
    t_layers: int = 5
    t_heads: int = 8
    t_hidden_scale: float = 4.0
    t_max_period: float = 10000.0
    t_weight_pos_embed: float = 1.0

    SOURCES = ("drums", "bass", "other", "vocals")

    @property
    def training_length(self) -> int:
        """`int(segment * samplerate)` (config.rs:222-224)."""
        return int(self.segment * self.samplerate)

    @property
    def hop_length(self) -> int:
        return self.nfft // 4

    def to_c(self) -> CConfig:
        return CConfig(**{f.name: getattr(self, f.name) for f in fields(self)})

    @classmethod
    def from_c(cls, c: CConfig) -> "Config":
        return cls(**{f.name: getattr(c, f.name) for f in fields(cls)})
