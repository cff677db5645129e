"""ctypes binding of libdmx.so (include/dmx.h, include/dmx_ops.h, include/dmx_ckpt.h).

The library is built in-tree by ``build.py`` (hipcc, gfx950). Loading fails
loudly when it is missing: there is no fallback implementation.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
LIBRARY_PATH = PACKAGE_DIR / "libdmx.so"

c_float_p = ctypes.POINTER(ctypes.c_float)
c_int64_p = ctypes.POINTER(ctypes.c_int64)
c_uint8_p = ctypes.POINTER(ctypes.c_uint8)

TRACE_WANTS = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_char_p, ctypes.c_void_p)
TRACE_RECORD = ctypes.CFUNCTYPE(None, ctypes.c_char_p, c_int64_p, ctypes.c_int32, c_float_p, ctypes.c_void_p)
PROGRESS = ctypes.CFUNCTYPE(None, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_void_p)
EMIT = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_int64, ctypes.c_int64, ctypes.POINTER(c_float_p), ctypes.c_void_p)


class CTensor(ctypes.Structure):
    _fields_ = [
        ("name", ctypes.c_char_p),
        ("data", c_float_p),
        ("ndim", ctypes.c_int32),
        ("shape", ctypes.c_int64 * 4),
    ]


class CAudioInfo(ctypes.Structure):
    _fields_ = [("sample_rate", ctypes.c_int32), ("channels", ctypes.c_int32), ("frames", ctypes.c_int64)]


class CComparison(ctypes.Structure):
    _fields_ = [
        ("elements", ctypes.c_int64),
        ("max_abs", ctypes.c_float),
        ("max_abs_index", ctypes.c_int64),
        ("max_rel", ctypes.c_float),
        ("mean_abs", ctypes.c_float),
        ("reference_max_abs", ctypes.c_float),
        ("reference_rms", ctypes.c_float),
        ("rms_relative_error", ctypes.c_float),
        ("snr_db", ctypes.c_float),
    ]


class CSeparateOptions(ctypes.Structure):
    _fields_ = [
        ("shifts", ctypes.c_int32),
        ("overlap", ctypes.c_double),
        ("transition_power", ctypes.c_double),
        ("segment", ctypes.c_double),
        ("batch_chunks", ctypes.c_int32),
    ]


# name -> (restype, argtypes). Every function declared in include/*.h appears
# here; tests check the library exports them all.
_VP, _I, _I64, _F, _D, _SZ = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_double, ctypes.c_size_t
SIGNATURES = {
    "dmx_config_default": (None, [_VP]),
    "dmx_config_training_length": (_I64, [_VP]),
    "dmx_last_error": (ctypes.c_char_p, []),
    "dmx_device_count": (_I, []),
    "dmx_runner_create": (_I, [ctypes.POINTER(CTensor), _SZ, _VP, _I, _I, ctypes.POINTER(_VP)]),
    "dmx_runner_destroy": (None, [_VP]),
    "dmx_runner_backend_tag": (ctypes.c_char_p, [_VP]),
    "dmx_runner_stream": (_VP, [_VP]),
    "dmx_synchronize": (_I, [_VP]),
    "dmx_forward_start": (_I, [_VP, _VP, _I64, _I64, _I64, ctypes.POINTER(_VP)]),
    "dmx_forward_collect": (_I, [_VP, _VP, _VP]),
    "dmx_forward": (_I, [_VP, _VP, _I64, _I64, _I64, _VP]),
    "dmx_forward_device": (_I, [_VP, _VP, _I64, _I64, _I64, _VP]),
    "dmx_crosstransformer_device": (_I, [_VP, _VP, _VP, _I64, _I64, _I64, _I64, _VP, _VP]),
    "dmx_set_trace": (_I, [_VP, TRACE_WANTS, TRACE_RECORD, _VP]),
    "dmx_separate_options_default": (None, [_VP]),
    "dmx_separate": (_I, [_VP, _VP, ctypes.c_int32, _VP, _VP, _VP, _I64, ctypes.c_int32, _VP, PROGRESS, _VP, _VP]),
    "dmx_separate_device": (_I, [_VP, _VP, ctypes.c_int32, _VP, _VP, _I64, ctypes.c_int32, _VP, PROGRESS, _VP, _VP]),
    "dmx_separate_emit": (_I, [_VP, _VP, ctypes.c_int32, _VP, _VP, _VP, _I64, ctypes.c_int32, _VP, PROGRESS, _VP,
                               EMIT, _VP]),
    # include/dmx_audio.h
    "dmx_audio_probe": (_I, [ctypes.c_char_p, ctypes.POINTER(CAudioInfo)]),
    "dmx_audio_read": (_I, [ctypes.c_char_p, _VP, _I64, ctypes.POINTER(CAudioInfo)]),
    "dmx_wav_write": (_I, [ctypes.c_char_p, _I, ctypes.c_int32, ctypes.c_int32, _VP, _I64]),
    "dmx_wav_writer_create": (_I, [ctypes.c_char_p, ctypes.c_int32, ctypes.c_int32, ctypes.POINTER(_VP)]),
    "dmx_wav_writer_write": (_I, [_VP, _VP, _I64]),
    "dmx_wav_writer_write_planar": (_I, [_VP, _VP, _I64, _I64]),
    "dmx_wav_writer_frames": (_I64, [_VP]),
    "dmx_wav_writer_finish": (_I, [_VP]),
    "dmx_compare": (_I, [_VP, _VP, _I64, ctypes.POINTER(CComparison)]),
    # include/dmx_ops.h
    "dmx_op_conv2d": (_I, [_VP, _VP, _VP] + [_I] * 4 + [_VP, _VP] + [_I] * 10 + [_VP]),
    "dmx_op_conv2d_glu": (_I, [_VP, _VP, _VP] + [_I] * 4 + [_VP, _VP] + [_I] * 5 + [_VP, _F, _VP]),
    "dmx_op_conv_transpose": (_I, [_VP, _VP] + [_I] * 4 + [_VP, _VP] + [_I] * 6 + [_VP]),
    "dmx_op_dconv_layer": (_I, [_VP, _VP] + [_I] * 5 + [_VP, _VP, _I] + [_VP] * 7),
    "dmx_op_dconv": (_I, [_VP, _VP] + [_I] * 5 + [_VP]),
    "dmx_op_linear": (_I, [_VP, _VP, _I, _I, _VP, _VP, _I, _I, _VP, _VP, _VP]),
    "dmx_op_pointwise": (_I, [_VP, _VP, _VP, _VP, _I, _I, _I, _I, _VP]),
    "dmx_op_attention": (_I, [_VP, _VP, _VP, _VP, _VP, _I, _I, _I, _I, _F]),
    "dmx_op_attention_pair": (_I, [_VP] + [_VP] * 4 + [_I, _I] + [_VP] * 4 + [_I, _I, _I, _I, _F]),
    "dmx_op_kv_planes": (_I, [_VP, _VP, _VP, _I, _I, _I, _VP, _VP]),
    "dmx_op_attention_pair_planes": (_I, [_VP] + [_VP] * 4 + [_I, _I] + [_VP] * 4 + [_I, _I, _I, _I, _F]),
    "dmx_op_layer_norm": (_I, [_VP, _VP, _I, _I, _VP, _VP, _VP]),
    "dmx_op_group_norm": (_I, [_VP, _VP, _I, _I, _I, _I, _VP, _VP, _VP]),
    "dmx_op_glu": (_I, [_VP, _VP, _I, _I, _I, _VP]),
    "dmx_op_gelu": (_I, [_VP, _VP, _I64, _VP]),
    "dmx_op_set_precision": (_I, [_I]),
    "dmx_op_spec_normalise": (_I, [_VP, _VP, _I, _I, _VP, _VP, _VP]),
    "dmx_op_spec_normalise_noalloc": (_I, [_VP, _VP, _I, _I, _VP, _VP, _VP]),
    "dmx_op_ispec_sum": (_I, [_VP, _VP, _VP, _I, _I, _VP, _VP]),
    # include/dmx_ckpt.h
    "dmx_checkpoint_load": (_I, [ctypes.c_char_p, ctypes.POINTER(_VP)]),
    "dmx_checkpoint_from_bytes": (_I, [_VP, _SZ, _I, ctypes.POINTER(_VP)]),
    "dmx_checkpoint_free": (None, [_VP]),
    "dmx_checkpoint_count": (_SZ, [_VP]),
    "dmx_checkpoint_tensors": (ctypes.POINTER(CTensor), [_VP]),
    "dmx_checkpoint_metadata": (ctypes.c_char_p, [_VP, ctypes.c_char_p]),
    "dmx_checkpoint_metadata_count": (_SZ, [_VP]),
    "dmx_checkpoint_metadata_key": (ctypes.c_char_p, [_VP, _SZ]),
    "dmx_checkpoint_config": (_I, [_VP, _VP]),
    "dmx_config_from_kwargs": (_I, [ctypes.c_char_p, _VP]),
}

_lib = None


class LibraryMissing(RuntimeError):
    pass


def load():
    """The loaded libdmx.so with every signature bound (cached)."""
    global _lib
    if _lib is not None:
        return _lib
    path = Path(os.environ.get("DMX_LIBRARY", LIBRARY_PATH))
    if not path.exists():
        raise LibraryMissing(f"{path} is not built; run __graft_entry__.build() (hipcc, gfx950) first")
    lib = ctypes.CDLL(str(path))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def last_error() -> str:
    msg = load().dmx_last_error()
    return msg.decode() if msg else ""
