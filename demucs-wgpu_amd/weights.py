"""Checkpoint key set, shapes and the seeded random-init recipe for HTDemucs v4.

The key names and shapes are the ones the reference loads
(crates/demucs-core/src/demucs/weights.rs:224-578 with the layer table of
crates/demucs-core/src/demucs/config.rs:325-444). No checkpoint ships here, so
every network is random-initialised by a counter-based generator (SplitMix64
per tensor, keyed by the tensor name and the seed), which makes the arrays
independent of numpy's RNG implementation and of generation order.

Recipe (``random_init``):
  * conv / linear weights and biases ~ U(-1/sqrt(fan_in), 1/sqrt(fan_in))
    (torch's default), fan_in = shape[1] * prod(shape[2:]) of the weight;
  * MultiheadAttention ``in_proj_weight`` ~ Xavier-uniform, ``in_proj_bias`` ~ U(-0.02, 0.02);
  * GroupNorm / LayerNorm weight ~ U(0.75, 1.25), bias ~ U(-0.2, 0.2) (not 1 / 0,
    so a dropped affine term fails parity);
  * LayerScale (``dconv...6.scale``, ``gamma_{1,2}.scale``) ~ U(0.1, 0.5), not the
    upstream 1e-3 init, so no branch is a near-identity a broken kernel could hide in;
  * ``freq_emb.embedding.weight`` ~ N(0, 1) (the loader then multiplies by emb_scale).
``xavier_transformer_init`` is the isolated-transformer recipe: Xavier-uniform
for every transformer matrix, the rest as above.
"""
from __future__ import annotations

import math
from collections import OrderedDict
from dataclasses import dataclass, field

import numpy as np

from .config import Config

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)


def _fnv1a64(text: str) -> int:
    h = 0xCBF29CE484222325
    for byte in text.encode():
        h ^= byte
        h = (h * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def _splitmix(z: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def stream_u01(key: str, seed: int, n: int) -> np.ndarray:
    """n uniforms in [0, 1) with 24-bit resolution from SplitMix64(key, seed)."""
    base = np.uint64((_fnv1a64(key) ^ ((seed * 0x9E3779B97F4A7C15) & 0xFFFFFFFFFFFFFFFF)) & 0xFFFFFFFFFFFFFFFF)
    with np.errstate(over="ignore"):
        counter = base + (np.arange(1, n + 1, dtype=np.uint64) * _GOLDEN)
    bits = _splitmix(counter) >> np.uint64(40)
    return bits.astype(np.float64) * (1.0 / (1 << 24))


def stream_uniform(key: str, seed: int, shape, lo: float, hi: float) -> np.ndarray:
    n = int(np.prod(shape))
    return (lo + (hi - lo) * stream_u01(key, seed, n)).astype(np.float32).reshape(shape)


def stream_normal(key: str, seed: int, shape, std: float = 1.0) -> np.ndarray:
    """Box-Muller over two independent uniform streams."""
    n = int(np.prod(shape))
    u1 = stream_u01(key + "#bm1", seed, n)
    u2 = stream_u01(key + "#bm2", seed, n)
    r = np.sqrt(-2.0 * np.log1p(-u1))  # 1 - u1 in (0, 1]
    return (std * r * np.cos(2.0 * math.pi * u2)).astype(np.float32).reshape(shape)


def weight_shapes(cfg: Config | None = None) -> "OrderedDict[str, tuple]":
    """Every tensor the reference loads, in checkpoint naming, with its shape."""
    c = cfg or Config()
    shapes: "OrderedDict[str, tuple]" = OrderedDict()
    hidden_div = 8

    def dconv(prefix: str, ch: int) -> None:
        hid = ch // hidden_div
        for d in range(2):
            at = f"{prefix}.layers.{d}"
            shapes[f"{at}.0.weight"] = (hid, ch, 3)
            shapes[f"{at}.0.bias"] = (hid,)
            shapes[f"{at}.1.weight"] = (hid,)
            shapes[f"{at}.1.bias"] = (hid,)
            shapes[f"{at}.3.weight"] = (2 * ch, hid, 1)
            shapes[f"{at}.3.bias"] = (2 * ch,)
            shapes[f"{at}.4.weight"] = (2 * ch,)
            shapes[f"{at}.4.bias"] = (2 * ch,)
            shapes[f"{at}.6.scale"] = (ch,)

    chin, chin_z = c.audio_channels, c.audio_channels * 2
    chout, chout_z = c.channels, c.channels
    freqs = c.nfft // 2
    dspec, tdspec = [], []
    freq_emb_rows = 0
    for i in range(c.depth):
        e, te = f"encoder.{i}", f"tencoder.{i}"
        shapes[f"{e}.conv.weight"] = (chout_z, chin_z, 8, 1)
        shapes[f"{e}.conv.bias"] = (chout_z,)
        shapes[f"{e}.rewrite.weight"] = (2 * chout_z, chout_z, 1, 1)
        shapes[f"{e}.rewrite.bias"] = (2 * chout_z,)
        dconv(f"{e}.dconv", chout_z)
        shapes[f"{te}.conv.weight"] = (chout, chin, 8)
        shapes[f"{te}.conv.bias"] = (chout,)
        shapes[f"{te}.rewrite.weight"] = (2 * chout, chout, 1)
        shapes[f"{te}.rewrite.bias"] = (2 * chout,)
        dconv(f"{te}.dconv", chout)
        if i == 0:
            chin = c.audio_channels * c.sources
            chin_z = chin * 2
        dspec.append((chout_z, chin_z))
        tdspec.append((chout, chin))
        if i == 0:
            freq_emb_rows = freqs // c.stride
        chin, chin_z = chout, chout_z
        chout *= c.growth
        chout_z *= c.growth
        freqs //= c.stride
    k = 1 + 2 * c.context
    for i in range(c.depth):
        d, td = f"decoder.{i}", f"tdecoder.{i}"
        ci, co = dspec[i]
        shapes[f"{d}.conv_tr.weight"] = (ci, co, 8, 1)
        shapes[f"{d}.conv_tr.bias"] = (co,)
        shapes[f"{d}.rewrite.weight"] = (2 * ci, ci, k, k)
        shapes[f"{d}.rewrite.bias"] = (2 * ci,)
        dconv(f"{d}.dconv", ci)
        ci, co = tdspec[i]
        shapes[f"{td}.conv_tr.weight"] = (ci, co, 8)
        shapes[f"{td}.conv_tr.bias"] = (co,)
        shapes[f"{td}.rewrite.weight"] = (2 * ci, ci, k)
        shapes[f"{td}.rewrite.bias"] = (2 * ci,)
        dconv(f"{td}.dconv", ci)
    pre = chin_z
    dim = c.bottom_channels
    hid = int(dim * c.t_hidden_scale)
    shapes["freq_emb.embedding.weight"] = (freq_emb_rows, c.channels)
    shapes["channel_upsampler.weight"] = (dim, pre, 1)
    shapes["channel_upsampler.bias"] = (dim,)
    shapes["channel_upsampler_t.weight"] = (dim, pre, 1)
    shapes["channel_upsampler_t.bias"] = (dim,)
    shapes["channel_downsampler.weight"] = (pre, dim, 1)
    shapes["channel_downsampler.bias"] = (pre,)
    shapes["channel_downsampler_t.weight"] = (pre, dim, 1)
    shapes["channel_downsampler_t.bias"] = (pre,)
    for nm in ("crosstransformer.norm_in", "crosstransformer.norm_in_t"):
        shapes[f"{nm}.weight"] = (dim,)
        shapes[f"{nm}.bias"] = (dim,)
    for i in range(c.t_layers):
        cross = i % 2 == 1
        for branch in ("layers", "layers_t"):
            p = f"crosstransformer.{branch}.{i}"
            a = f"{p}.{'cross_attn' if cross else 'self_attn'}"
            shapes[f"{a}.in_proj_weight"] = (3 * dim, dim)
            shapes[f"{a}.in_proj_bias"] = (3 * dim,)
            shapes[f"{a}.out_proj.weight"] = (dim, dim)
            shapes[f"{a}.out_proj.bias"] = (dim,)
            shapes[f"{p}.linear1.weight"] = (hid, dim)
            shapes[f"{p}.linear1.bias"] = (hid,)
            shapes[f"{p}.linear2.weight"] = (dim, hid)
            shapes[f"{p}.linear2.bias"] = (dim,)
            for nm in ["norm1", "norm2"] + (["norm3"] if cross else []) + ["norm_out"]:
                shapes[f"{p}.{nm}.weight"] = (dim,)
                shapes[f"{p}.{nm}.bias"] = (dim,)
            shapes[f"{p}.gamma_1.scale"] = (dim,)
            shapes[f"{p}.gamma_2.scale"] = (dim,)
    return shapes


def _is_norm(name: str) -> bool:
    parts = name.split(".")
    if "norm" in parts[-2] or parts[-2] in ("norm_in", "norm_in_t"):
        return True
    # DConv GroupNorms are modules 1 and 4 of the branch.
    return ".dconv.layers." in name and parts[-2] in ("1", "4")


def _fan_in(shape: tuple) -> int:
    return int(shape[1] * int(np.prod(shape[2:]))) if len(shape) >= 2 else int(shape[0])


def random_init(seed: int, cfg: Config | None = None, xavier_transformer: bool = False) -> "OrderedDict[str, np.ndarray]":
    """Seeded random weights for every tensor of ``weight_shapes(cfg)``."""
    shapes = weight_shapes(cfg)
    out: "OrderedDict[str, np.ndarray]" = OrderedDict()
    for name, shape in shapes.items():
        key = name
        if name.endswith(".scale"):
            out[name] = stream_uniform(key, seed, shape, 0.1, 0.5)
        elif name == "freq_emb.embedding.weight":
            out[name] = stream_normal(key, seed, shape)
        elif _is_norm(name):
            if name.endswith(".weight"):
                out[name] = stream_uniform(key, seed, shape, 0.75, 1.25)
            else:
                out[name] = stream_uniform(key, seed, shape, -0.2, 0.2)
        elif name.endswith("in_proj_weight"):
            bound = math.sqrt(6.0 / (shape[0] + shape[1]))
            out[name] = stream_uniform(key, seed, shape, -bound, bound)
        elif name.endswith("in_proj_bias"):
            out[name] = stream_uniform(key, seed, shape, -0.02, 0.02)
        elif name.endswith(".weight"):
            if xavier_transformer and name.startswith("crosstransformer."):
                fan_out = shape[0] * int(np.prod(shape[2:]))
                bound = math.sqrt(6.0 / (_fan_in(shape) + fan_out))
            else:
                bound = 1.0 / math.sqrt(_fan_in(shape))
            out[name] = stream_uniform(key, seed, shape, -bound, bound)
        elif name.endswith(".bias"):
            wshape = shapes[name[: -len(".bias")] + ".weight"]
            bound = 1.0 / math.sqrt(_fan_in(wshape))
            if xavier_transformer and name.startswith("crosstransformer."):
                bound = 0.02
            out[name] = stream_uniform(key, seed, shape, -bound, bound)
        else:  # pragma: no cover - every key is handled above
            raise KeyError(name)
    return out


def xavier_transformer_init(seed: int, cfg: Config | None = None) -> "OrderedDict[str, np.ndarray]":
    return random_init(seed, cfg, xavier_transformer=True)


def parameter_count(weights) -> int:
    return int(sum(int(np.prod(v.shape)) for v in weights.values()))
