"""ctypes binding of oracle/liboracle.so — the CPU restatement of the reference's
host backend.

TEST INFRASTRUCTURE ONLY: imported by tests/, `__graft_entry__.smoke()` and
bench.py's cpu_baseline leg, as the checker. The product package never
imports this module.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path
from typing import Callable, Dict, Mapping, Optional, Sequence, Tuple

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
LIBRARY = ORACLE_DIR / "liboracle.so"

_VP, _I, _I32, _I64, _F, _D = ctypes.c_void_p, ctypes.c_int, ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_double
FWD = ctypes.CFUNCTYPE(_I, _VP, _I64, _I64, _I64, _VP, _VP)
WANTS = ctypes.CFUNCTYPE(_I, ctypes.c_char_p, _VP)
RECORD = ctypes.CFUNCTYPE(None, ctypes.c_char_p, ctypes.POINTER(_I64), _I32, ctypes.POINTER(_F), _VP)

_SIG = {
    "oracle_last_error": (ctypes.c_char_p, []),
    "oracle_set_threads": (None, [_I]),
    "oracle_get_threads": (_I, []),
    "oracle_sgemm": (None, [_I64, _I64, _I64, _VP, _I64, _I64, _VP, _I64, _I64, _VP, _I64]),
    "oracle_conv2d": (_I, [_VP, _I64, _I64, _I64, _I64, _VP, _VP] + [_I64] * 9 + [_VP]),
    "oracle_conv_transpose2d": (_I, [_VP, _I64, _I64, _I64, _I64, _VP, _VP] + [_I64] * 5 + [_VP]),
    "oracle_group_norm": (_I, [_VP, _I64, _I64, _I64, _I64, _VP, _VP, _VP]),
    "oracle_group_norm_glu": (_I, [_VP, _I64, _I64, _I64, _I64, _VP, _VP, _VP]),
    "oracle_layer_norm_rows": (_I, [_VP, _I64, _I64, _VP, _VP, _VP]),
    "oracle_glu": (_I, [_VP, _I64, _I64, _I64, _VP]),
    "oracle_gelu": (None, [_VP, _I64, _VP]),
    "oracle_gelu_scalar": (_F, [_F]),
    "oracle_mean": (_F, [_VP, _I64]),
    "oracle_std_unbiased": (_F, [_VP, _I64]),
    "oracle_attention_head": (_I, [_VP, _VP, _VP, _I64, _I64, _I64, _F, _VP]),
    "oracle_multi_head_attention": (_I, [_VP, _VP, _I64, _I64, _I64, _I64, _I64] + [_VP] * 8 + [_VP]),
    "oracle_dconv": (_I, [_VP, _I64, _I64, _I64, _VP, ctypes.c_size_t, ctypes.c_char_p, _VP]),
    "oracle_hann_window": (None, [_I64, _VP]),
    "oracle_fft": (None, [_VP, _VP, _I64, _I, _VP, _VP]),
    "oracle_stft": (_I, [_VP, _I64, _I64, _I64, _I64, _I, _VP, _VP, ctypes.POINTER(_I64)]),
    "oracle_istft": (_I, [_VP, _VP, _I64, _I64, _I64, _I64, _I64, _I, _I64, _VP, ctypes.POINTER(_I64)]),
    "oracle_pad1d_reflect": (_I, [_VP, _I64, _I64, _I64, _VP]),
    "oracle_spec_cac": (_I, [_VP, _I64, _I64, _I64, _I64, _VP]),
    "oracle_ispec_cac": (_I, [_VP, _I64, _I64, _I64, _I64, _I64, _I64, _VP]),
    "oracle_positions_2d": (None, [_I64, _I64, _I64, _F, _VP]),
    "oracle_positions_1d": (None, [_I64, _I64, _F, _VP]),
    "oracle_transition_weight": (None, [_I64, _D, _VP]),
    "oracle_shift_rng": (None, [ctypes.c_uint64, _I64, _I64, _VP]),
    "oracle_scan_norm": (None, [_VP, _I64, _I64, _I64, ctypes.POINTER(_F), ctypes.POINTER(_F)]),
    "oracle_model_create": (_VP, [_VP, ctypes.c_size_t, _VP]),
    "oracle_model_destroy": (None, [_VP]),
    "oracle_model_training_length": (_I64, [_VP]),
    "oracle_forward": (_I, [_VP, _VP, _I64, _I64, _I64, _VP, WANTS, RECORD, _VP]),
    "oracle_transformer_forward": (_I, [_VP, _VP, _VP, _I64, _I64, _I64, _I64, _VP, _VP, WANTS, RECORD, _VP]),
    "oracle_separate": (_I, [_VP, _VP, _I32, _VP, _VP, _VP, _I64, _I32, _VP, FWD, _VP, _I32, _VP]),
    "oracle_split_pass": (_I, [_VP, _I64, _I64, _I64, _I64, _D, _D, _I64, _I64, _I32, _I32, FWD, _VP, _VP]),
}

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", str(ORACLE_DIR)], check=True)


def lib():
    global _lib
    if _lib is None:
        if not LIBRARY.exists():
            build()
        l = ctypes.CDLL(str(LIBRARY))
        for name, (res, args) in _SIG.items():
            fn = getattr(l, name)
            fn.restype = res
            fn.argtypes = args
        _lib = l
    return _lib


class OracleError(RuntimeError):
    pass


def _check(rc: int) -> None:
    if rc != 0:
        raise OracleError(lib().oracle_last_error().decode())


def f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def p(a: Optional[np.ndarray]):
    return None if a is None else ctypes.c_void_p(a.ctypes.data)


def set_threads(n: int) -> None:
    lib().oracle_set_threads(n)


def threads() -> int:
    return lib().oracle_get_threads()


# ---- operators ----

def sgemm(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a, b = f32(a), f32(b)
    m, k = a.shape
    n = b.shape[1]
    c = np.empty((m, n), np.float32)
    lib().oracle_sgemm(m, n, k, p(a), k, 1, p(b), n, 1, p(c), n)
    return c


def conv2d(x, w, bias, stride=(1, 1), pad=(0, 0), dilation=(1, 1)) -> np.ndarray:
    x, w = f32(x), f32(w)
    bias = None if bias is None else f32(bias)
    b, ic, h, wd = x.shape
    oc, _, kh, kw = w.shape
    eh, ew = dilation[0] * (kh - 1) + 1, dilation[1] * (kw - 1) + 1
    oh = (h + 2 * pad[0] - eh) // stride[0] + 1
    ow = (wd + 2 * pad[1] - ew) // stride[1] + 1
    out = np.empty((b, oc, oh, ow), np.float32)
    _check(lib().oracle_conv2d(p(x), b, ic, h, wd, p(w), p(bias), oc, kh, kw, stride[0], stride[1], pad[0], pad[1],
                               dilation[0], dilation[1], p(out)))
    return out


def conv1d(x, w, bias, stride=1, pad=0, dilation=1) -> np.ndarray:
    x, w = f32(x), f32(w)
    out = conv2d(x[:, :, None, :], w[:, :, None, :], bias, (1, stride), (0, pad), (1, dilation))
    return out[:, :, 0, :]


def conv_transpose2d(x, w, bias, stride=(1, 1)) -> np.ndarray:
    x, w = f32(x), f32(w)
    bias = None if bias is None else f32(bias)
    b, ic, h, wd = x.shape
    _, oc, kh, kw = w.shape
    out = np.empty((b, oc, (h - 1) * stride[0] + kh, (wd - 1) * stride[1] + kw), np.float32)
    _check(lib().oracle_conv_transpose2d(p(x), b, ic, h, wd, p(w), p(bias), oc, kh, kw, stride[0], stride[1], p(out)))
    return out


def conv_transpose1d(x, w, bias, stride=1) -> np.ndarray:
    return conv_transpose2d(f32(x)[:, :, None, :], f32(w)[:, :, None, :], bias, (1, stride))[:, :, 0, :]


def group_norm(x, groups, w, b) -> np.ndarray:
    x = f32(x)
    out = np.empty_like(x)
    inner = int(np.prod(x.shape[2:])) if x.ndim > 2 else 1
    w, b = f32(w), f32(b)
    _check(lib().oracle_group_norm(p(x), x.shape[0], x.shape[1], inner, groups, p(w), p(b), p(out)))
    return out


def group_norm_glu(x, groups, w, b) -> np.ndarray:
    x = f32(x)
    shape = list(x.shape)
    shape[1] //= 2
    out = np.empty(shape, np.float32)
    inner = int(np.prod(x.shape[2:])) if x.ndim > 2 else 1
    w, b = f32(w), f32(b)
    _check(lib().oracle_group_norm_glu(p(x), x.shape[0], x.shape[1], inner, groups, p(w), p(b), p(out)))
    return out


def layer_norm(x, w, b) -> np.ndarray:
    x = f32(x)
    out = np.empty_like(x)
    dim = x.shape[-1]
    w, b = f32(w), f32(b)
    _check(lib().oracle_layer_norm_rows(p(x), x.size // dim, dim, p(w), p(b), p(out)))
    return out


def glu(x) -> np.ndarray:
    x = f32(x)
    shape = list(x.shape)
    shape[1] //= 2
    out = np.empty(shape, np.float32)
    inner = int(np.prod(x.shape[2:])) if x.ndim > 2 else 1
    _check(lib().oracle_glu(p(x), x.shape[0], x.shape[1], inner, p(out)))
    return out


def gelu(x) -> np.ndarray:
    x = f32(x)
    out = np.empty_like(x)
    lib().oracle_gelu(p(x), x.size, p(out))
    return out


def mean(x) -> float:
    x = f32(x)
    return lib().oracle_mean(p(x), x.size)


def std_unbiased(x) -> float:
    x = f32(x)
    return lib().oracle_std_unbiased(p(x), x.size)


def attention_head(q, k, v, scale) -> np.ndarray:
    q, k, v = f32(q), f32(k), f32(v)
    out = np.empty((q.shape[0], q.shape[1]), np.float32)
    _check(lib().oracle_attention_head(p(q), p(k), p(v), q.shape[0], k.shape[0], q.shape[1], scale, p(out)))
    return out


def multi_head_attention(query, key, heads, wq, bq, wk, bk, wv, bv, wo, bo) -> np.ndarray:
    query, key = f32(query), f32(key)
    b, nq, dim = query.shape
    nk = key.shape[1]
    out = np.empty_like(query)
    args = [f32(t) for t in (wq, bq, wk, bk, wv, bv, wo, bo)]
    _check(lib().oracle_multi_head_attention(p(query), p(key), b, nq, nk, dim, heads, *[p(t) for t in args], p(out)))
    return out


def _tensors(weights: Mapping[str, np.ndarray]):
    """Build the dmx_tensor array (keeps references alive in the returned tuple)."""
    from ctypes import Structure, POINTER, c_char_p, c_int32, c_int64, c_float

    class CTensor(Structure):
        _fields_ = [("name", c_char_p), ("data", POINTER(c_float)), ("ndim", c_int32), ("shape", c_int64 * 4)]

    arrays = [(k.encode(), f32(v)) for k, v in weights.items()]
    entries = (CTensor * len(arrays))()
    for i, (name, arr) in enumerate(arrays):
        entries[i].name = name
        entries[i].data = arr.ctypes.data_as(POINTER(c_float))
        entries[i].ndim = arr.ndim
        for d in range(arr.ndim):
            entries[i].shape[d] = arr.shape[d]
    return entries, arrays


def dconv(x, weights: Mapping[str, np.ndarray], prefix: str) -> np.ndarray:
    x = f32(x)
    entries, keep = _tensors(weights)
    out = np.empty_like(x)
    _check(lib().oracle_dconv(p(x), x.shape[0], x.shape[1], x.shape[2], ctypes.cast(entries, _VP), len(keep),
                              prefix.encode(), p(out)))
    return out


def hann_window(n: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().oracle_hann_window(n, p(out))
    return out


def fft(x: np.ndarray, inverse: bool = False) -> np.ndarray:
    x = np.asarray(x)
    re = f32(x.real)
    im = f32(x.imag) if np.iscomplexobj(x) else np.zeros_like(re)
    orr, oi = np.empty(re.size), np.empty(re.size)
    lib().oracle_fft(p(re), p(im), re.size, 1 if inverse else 0, p(orr), p(oi))
    return orr + 1j * oi


def stft(x, n_fft, hop, normalized=False) -> np.ndarray:
    x = f32(x)
    batch, samples = x.shape
    frames = ctypes.c_int64()
    _check(lib().oracle_stft(p(x), batch, samples, n_fft, hop, int(normalized), None, None, ctypes.byref(frames)))
    bins = n_fft // 2 + 1
    re = np.empty((batch, bins, frames.value), np.float32)
    im = np.empty_like(re)
    _check(lib().oracle_stft(p(x), batch, samples, n_fft, hop, int(normalized), p(re), p(im), ctypes.byref(frames)))
    return re + 1j * im


def istft(spec, n_fft, hop, normalized=False, length: Optional[int] = None) -> np.ndarray:
    re, im = f32(np.real(spec)), f32(np.imag(spec))
    batch, bins, frames = re.shape
    n = ctypes.c_int64()
    ln = -1 if length is None else length
    _check(lib().oracle_istft(p(re), p(im), batch, bins, frames, n_fft, hop, int(normalized), ln, None, ctypes.byref(n)))
    out = np.empty((batch, n.value), np.float32)
    _check(lib().oracle_istft(p(re), p(im), batch, bins, frames, n_fft, hop, int(normalized), ln, p(out), ctypes.byref(n)))
    return out


def pad1d_reflect(x, left, right) -> np.ndarray:
    x = f32(x)
    out = np.empty(x.size + left + right, np.float32)
    _check(lib().oracle_pad1d_reflect(p(x), x.size, left, right, p(out)))
    return out


def spec_cac(mix, nfft=4096) -> np.ndarray:
    mix = f32(mix)
    b, c, n = mix.shape
    le = -(-n // (nfft // 4))
    out = np.empty((b, 2 * c, nfft // 2, le), np.float32)
    _check(lib().oracle_spec_cac(p(mix), b, c, n, nfft, p(out)))
    return out


def ispec_cac(x, sources, length, nfft=4096) -> np.ndarray:
    x = f32(x)
    b, ch, fr, le = x.shape
    out = np.empty((b, sources, 2, length), np.float32)
    _check(lib().oracle_ispec_cac(p(x), b, sources, fr, le, nfft, length, p(out)))
    return out


def positions_2d(dim, height, width, max_period=10000.0) -> np.ndarray:
    out = np.empty((width * height, dim), np.float32)
    lib().oracle_positions_2d(dim, height, width, max_period, p(out))
    return out


def positions_1d(length, dim, max_period=10000.0) -> np.ndarray:
    out = np.empty((length, dim), np.float32)
    lib().oracle_positions_1d(length, dim, max_period, p(out))
    return out


def transition_weight(n, power=1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().oracle_transition_weight(n, power, p(out))
    return out


def shift_rng(seed: int, max_value: int, count: int) -> np.ndarray:
    out = np.empty(count, np.int64)
    lib().oracle_shift_rng(seed, max_value, count, p(out))
    return out


def scan_norm(wav) -> Tuple[float, float]:
    wav = f32(wav)
    m, s = ctypes.c_float(), ctypes.c_float()
    lib().oracle_scan_norm(p(wav), wav.shape[0], wav.shape[1], wav.shape[2], ctypes.byref(m), ctypes.byref(s))
    return m.value, s.value


# ---- the model ----

class Model:
    def __init__(self, weights: Mapping[str, np.ndarray], config=None):
        from importlib import import_module
        cfg = config
        if cfg is None:
            cfg = _default_cconfig()
        elif hasattr(cfg, "to_c"):
            cfg = cfg.to_c()
        self._cfg = cfg
        entries, keep = _tensors(weights)
        h = lib().oracle_model_create(ctypes.cast(entries, _VP), len(keep), ctypes.byref(cfg))
        if not h:
            raise OracleError(lib().oracle_last_error().decode())
        self.handle = ctypes.c_void_p(h)

    def __del__(self):
        if getattr(self, "handle", None):
            lib().oracle_model_destroy(self.handle)
            self.handle = None

    @property
    def training_length(self) -> int:
        return lib().oracle_model_training_length(self.handle)

    def forward(self, mix, trace: Optional[Dict[str, np.ndarray]] = None,
                wants: Optional[Callable[[str], bool]] = None) -> np.ndarray:
        mix = f32(mix)
        b, c, n = mix.shape
        out = np.empty((b, 4, c, n), np.float32)
        w, r = _trace_callbacks(trace, wants)
        _check(lib().oracle_forward(self.handle, p(mix), b, c, n, p(out), w, r, None))
        return out

    def transformer(self, x, xt, trace=None, wants=None):
        x, xt = f32(x), f32(xt)
        b, d, f, t = x.shape
        lt = xt.shape[2]
        xo, xto = np.empty_like(x), np.empty_like(xt)
        w, r = _trace_callbacks(trace, wants)
        _check(lib().oracle_transformer_forward(self.handle, p(x), p(xt), b, f, t, lt, p(xo), p(xto), w, r, None))
        return xo, xto


def _trace_callbacks(trace, wants):
    if trace is None:
        return WANTS(), RECORD()

    def _w(name, _u):
        return 1 if (wants is None or wants(name.decode())) else 0

    def _r(name, shape, ndim, data, _u):
        dims = tuple(shape[i] for i in range(ndim))
        trace[name.decode()] = np.ctypeslib.as_array(data, shape=(int(np.prod(dims)),)).copy().reshape(dims)

    cbs = (WANTS(_w), RECORD(_r))
    _trace_callbacks.keep = cbs  # keep alive for the duration of the call
    return cbs


def _default_cconfig():
    import sys
    pkg = sys.modules.get("demucs_wgpu_amd")
    if pkg is not None:
        return pkg.Config().to_c()
    raise OracleError("pass a config (demucs_wgpu_amd.Config) explicitly")


def separate(models: Sequence[Model], left, right, sample_rate, options, bag_weights=None, wanted=None,
             forward: Optional[Callable[[np.ndarray], np.ndarray]] = None, sources: int = 4) -> np.ndarray:
    """oracle_separate: (sources, 2, samples)."""
    left, right = f32(left), f32(right)
    out = np.zeros((sources, 2, left.size), np.float32)
    handles = (ctypes.c_void_p * max(1, len(models)))(*[m.handle for m in models])
    w = None if bag_weights is None else f32(bag_weights)
    mask = None if wanted is None else np.array([1 if x else 0 for x in wanted], np.uint8)
    opts = options.to_c()
    cb = FWD()
    if forward is not None:
        def _fwd(padded, b, c, n, outp, _u):
            arr = np.ctypeslib.as_array(ctypes.cast(padded, ctypes.POINTER(ctypes.c_float)), shape=(b * c * n,))
            res = f32(forward(arr.reshape(b, c, n).copy()))
            ctypes.memmove(outp, res.ctypes.data, res.nbytes)
            return 0
        cb = FWD(_fwd)
    _check(lib().oracle_separate(handles, p(w), len(models), p(mask), p(left), p(right), left.size, sample_rate,
                                 ctypes.byref(opts), cb, None, sources, p(out)))
    return out


def split_pass(mix, segment_length, overlap, power, shift_offset, max_shift, batch_chunks, sources,
               forward: Callable[[np.ndarray], np.ndarray]) -> np.ndarray:
    mix = f32(mix)
    b, c, n = mix.shape
    view = n + max_shift - shift_offset if max_shift > 0 else n
    out = np.empty((b, sources, c, view), np.float32)

    def _fwd(padded, bb, cc, nn, outp, _u):
        arr = np.ctypeslib.as_array(ctypes.cast(padded, ctypes.POINTER(ctypes.c_float)), shape=(bb * cc * nn,))
        res = f32(forward(arr.reshape(bb, cc, nn).copy()))
        ctypes.memmove(outp, res.ctypes.data, res.nbytes)
        return 0

    cb = FWD(_fwd)
    _check(lib().oracle_split_pass(p(mix), b, c, n, segment_length, overlap, power, shift_offset, max_shift,
                                   batch_chunks, sources, cb, None, p(out)))
    return out
