"""Checkpoint loading through the native readers of include/dmx_ckpt.h.

`load_weights(path)` mirrors the reference's `load_weights`
(crates/demucs-core/src/demucs/weights.rs:56-88): ``.th`` / ``.pth`` / ``.pt``
files are torch.save zips read by a data-only pickle interpreter, anything else
is safetensors; the config comes from the safetensors ``kwargs`` metadata when
present and is `HtdemucsConfig::default` otherwise. `load_weights_from_bytes`
mirrors `load_weights_from_bytes` (weights.rs:30-50).
"""
from __future__ import annotations

import ctypes
import os
from collections import OrderedDict
from dataclasses import dataclass, field
from typing import Dict, Union

import numpy as np

from . import _native
from .config import CConfig, Config


@dataclass
class LoadedWeights:
    """`LoadedWeights` (weights.rs:20-27): tensors by checkpoint name (f32,
    sorted by name), the model config and the safetensors metadata."""

    tensors: "OrderedDict[str, np.ndarray]"
    config: Config
    metadata: Dict[str, str] = field(default_factory=dict)


class CheckpointError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


def _check(rc: int) -> None:
    if rc != 0:
        raise CheckpointError(rc, _native.last_error())


def _collect(lib, handle: ctypes.c_void_p) -> LoadedWeights:
    try:
        n = lib.dmx_checkpoint_count(handle)
        entries = lib.dmx_checkpoint_tensors(handle)
        tensors: "OrderedDict[str, np.ndarray]" = OrderedDict()
        for i in range(n):
            e = entries[i]
            shape = tuple(int(e.shape[d]) for d in range(e.ndim))
            count = int(np.prod(shape, dtype=np.int64)) if shape else 1
            if count:
                flat = np.ctypeslib.as_array(e.data, shape=(count,))
                tensors[e.name.decode()] = flat.reshape(shape).copy()
            else:
                tensors[e.name.decode()] = np.zeros(shape, np.float32)
        metadata = {}
        for i in range(lib.dmx_checkpoint_metadata_count(handle)):
            key = lib.dmx_checkpoint_metadata_key(handle, i)
            metadata[key.decode()] = lib.dmx_checkpoint_metadata(handle, key).decode()
        c = CConfig()
        _check(lib.dmx_checkpoint_config(handle, ctypes.byref(c)))
        return LoadedWeights(tensors, Config.from_c(c), metadata)
    finally:
        lib.dmx_checkpoint_free(handle)


def load_weights(path: Union[str, os.PathLike]) -> LoadedWeights:
    lib = _native.load()
    handle = ctypes.c_void_p()
    _check(lib.dmx_checkpoint_load(os.fsencode(path), ctypes.byref(handle)))
    return _collect(lib, handle)


def load_weights_from_bytes(data: bytes, torch_zip: bool) -> LoadedWeights:
    lib = _native.load()
    handle = ctypes.c_void_p()
    buf = ctypes.create_string_buffer(bytes(data), len(data))
    _check(lib.dmx_checkpoint_from_bytes(buf, len(data), 1 if torch_zip else 0, ctypes.byref(handle)))
    return _collect(lib, handle)


def config_from_kwargs(text: str) -> Config:
    """`HtdemucsConfig::from_kwargs_json` (config.rs:150-215)."""
    lib = _native.load()
    c = CConfig()
    _check(lib.dmx_config_from_kwargs(text.encode(), ctypes.byref(c)))
    return Config.from_c(c)
