"""An independent float64 torch composition of HTDemucs v4's forward, used only
to pin the CPU oracle.

It is written from the upstream model's PyTorch semantics (torch.stft/istft
with normalized=True, nn.Conv*/ConvTranspose*, F.group_norm, F.layer_norm,
nn.MultiheadAttention math, exact F.gelu) — not from the oracle's code — so an
index, sign or operand mistake in the oracle shows up as a large error here.
Everything runs in float64 on the CPU.
"""
import math

import numpy as np
import torch
import torch.nn.functional as F

DT = torch.float64


def T(a):
    return torch.as_tensor(np.asarray(a), dtype=DT)


class Weights:
    def __init__(self, w):
        self.w = {k: T(v) for k, v in w.items()}

    def __getitem__(self, k):
        return self.w[k]


def dconv(W, prefix, x):
    """DConv on (N, C, T): two residual layers, dilation 1 and 2."""
    for d in range(2):
        at = f"{prefix}.layers.{d}"
        dil = 2 ** d
        y = F.conv1d(x, W[f"{at}.0.weight"], W[f"{at}.0.bias"], padding=dil, dilation=dil)
        y = F.group_norm(y, 1, W[f"{at}.1.weight"], W[f"{at}.1.bias"], eps=1e-5)
        y = F.gelu(y)
        y = F.conv1d(y, W[f"{at}.3.weight"], W[f"{at}.3.bias"])
        y = F.group_norm(y, 1, W[f"{at}.4.weight"], W[f"{at}.4.bias"], eps=1e-5)
        y = F.glu(y, dim=1)
        y = W[f"{at}.6.scale"][:, None] * y
        x = x + y
    return x


def enc_freq(W, i, x):
    p = f"encoder.{i}"
    y = F.gelu(F.conv2d(x, W[f"{p}.conv.weight"], W[f"{p}.conv.bias"], stride=(4, 1), padding=(2, 0)))
    B, C, Fr, Tn = y.shape
    y = y.permute(0, 2, 1, 3).reshape(-1, C, Tn)
    y = dconv(W, f"{p}.dconv", y)
    y = y.view(B, Fr, C, Tn).permute(0, 2, 1, 3)
    z = F.conv2d(y, W[f"{p}.rewrite.weight"], W[f"{p}.rewrite.bias"])
    return F.glu(z, dim=1)


def enc_time(W, i, x):
    p = f"tencoder.{i}"
    le = x.shape[-1]
    if le % 4:
        x = F.pad(x, (0, 4 - le % 4))
    y = F.gelu(F.conv1d(x, W[f"{p}.conv.weight"], W[f"{p}.conv.bias"], stride=4, padding=2))
    y = dconv(W, f"{p}.dconv", y)
    z = F.conv1d(y, W[f"{p}.rewrite.weight"], W[f"{p}.rewrite.bias"])
    return F.glu(z, dim=1)


def dec_freq(W, i, x, skip, last):
    p = f"decoder.{i}"
    x = x + skip
    y = F.glu(F.conv2d(x, W[f"{p}.rewrite.weight"], W[f"{p}.rewrite.bias"], padding=1), dim=1)
    B, C, Fr, Tn = y.shape
    y = y.permute(0, 2, 1, 3).reshape(-1, C, Tn)
    y = dconv(W, f"{p}.dconv", y)
    y = y.view(B, Fr, C, Tn).permute(0, 2, 1, 3)
    z = F.conv_transpose2d(y, W[f"{p}.conv_tr.weight"], W[f"{p}.conv_tr.bias"], stride=(4, 1))
    z = z[..., 2:-2, :]
    return z if last else F.gelu(z)


def dec_time(W, i, x, skip, length, last):
    p = f"tdecoder.{i}"
    x = x + skip
    y = F.glu(F.conv1d(x, W[f"{p}.rewrite.weight"], W[f"{p}.rewrite.bias"], padding=1), dim=1)
    y = dconv(W, f"{p}.dconv", y)
    z = F.conv_transpose1d(y, W[f"{p}.conv_tr.weight"], W[f"{p}.conv_tr.bias"], stride=4)
    z = z[..., 2:2 + length]
    return z if last else F.gelu(z)


def sin_2d(d_model, height, width, max_period=10000.0):
    pe = torch.zeros(d_model, height, width, dtype=DT)
    half = d_model // 2
    div = torch.exp(torch.arange(0.0, half, 2, dtype=DT) * -(math.log(max_period) / half))
    pos_w = torch.arange(0.0, width, dtype=DT).unsqueeze(1)
    pos_h = torch.arange(0.0, height, dtype=DT).unsqueeze(1)
    pe[0:half:2] = torch.sin(pos_w * div).transpose(0, 1).unsqueeze(1).repeat(1, height, 1)
    pe[1:half:2] = torch.cos(pos_w * div).transpose(0, 1).unsqueeze(1).repeat(1, height, 1)
    pe[half::2] = torch.sin(pos_h * div).transpose(0, 1).unsqueeze(2).repeat(1, 1, width)
    pe[half + 1::2] = torch.cos(pos_h * div).transpose(0, 1).unsqueeze(2).repeat(1, 1, width)
    return pe[None]


def sin_1d(length, dim, max_period=10000.0):
    pos = torch.arange(length, dtype=DT).view(-1, 1)
    half = dim // 2
    adim = torch.arange(half, dtype=DT).view(1, -1)
    phase = pos / (max_period ** (adim / (half - 1)))
    return torch.cat([torch.cos(phase), torch.sin(phase)], dim=-1)  # (T, C)


def mha(W, prefix, q, k, heads):
    wi, bi = W[f"{prefix}.in_proj_weight"], W[f"{prefix}.in_proj_bias"]
    D = q.shape[-1]
    Q = q @ wi[:D].T + bi[:D]
    K = k @ wi[D:2 * D].T + bi[D:2 * D]
    V = k @ wi[2 * D:].T + bi[2 * D:]
    B, Lq, _ = Q.shape
    Lk = K.shape[1]
    dh = D // heads
    Q = Q.view(B, Lq, heads, dh).transpose(1, 2)
    K = K.view(B, Lk, heads, dh).transpose(1, 2)
    V = V.view(B, Lk, heads, dh).transpose(1, 2)
    att = torch.softmax(Q @ K.transpose(-1, -2) / math.sqrt(dh), dim=-1)
    O = (att @ V).transpose(1, 2).reshape(B, Lq, D)
    return O @ W[f"{prefix}.out_proj.weight"].T + W[f"{prefix}.out_proj.bias"]


def ff(W, p, x):
    h = F.gelu(x @ W[f"{p}.linear1.weight"].T + W[f"{p}.linear1.bias"])
    return h @ W[f"{p}.linear2.weight"].T + W[f"{p}.linear2.bias"]


def ln(W, name, x):
    return F.layer_norm(x, (x.shape[-1],), W[f"{name}.weight"], W[f"{name}.bias"], eps=1e-5)


def gn_out(W, p, x):
    y = F.group_norm(x.transpose(1, 2), 1, W[f"{p}.norm_out.weight"], W[f"{p}.norm_out.bias"], eps=1e-5)
    return y.transpose(1, 2)


def self_layer(W, p, x, heads):
    x = x + W[f"{p}.gamma_1.scale"] * mha(W, f"{p}.self_attn", ln(W, f"{p}.norm1", x), ln(W, f"{p}.norm1", x), heads)
    x = x + W[f"{p}.gamma_2.scale"] * ff(W, p, ln(W, f"{p}.norm2", x))
    return gn_out(W, p, x)


def cross_layer(W, p, q, k, heads):
    x = q + W[f"{p}.gamma_1.scale"] * mha(W, f"{p}.cross_attn", ln(W, f"{p}.norm1", q), ln(W, f"{p}.norm2", k), heads)
    x = x + W[f"{p}.gamma_2.scale"] * ff(W, p, ln(W, f"{p}.norm3", x))
    return gn_out(W, p, x)


def transformer(W, x, xt, layers=5, heads=8, trace=None):
    B, C, Fr, T1 = x.shape
    pos = sin_2d(C, Fr, T1).permute(0, 3, 2, 1).reshape(1, T1 * Fr, C)
    x = x.permute(0, 3, 2, 1).reshape(B, T1 * Fr, C)
    x = ln(W, "crosstransformer.norm_in", x) + pos
    T2 = xt.shape[-1]
    xt = xt.transpose(1, 2)
    xt = ln(W, "crosstransformer.norm_in_t", xt) + sin_1d(T2, C)[None]
    for i in range(layers):
        p, pt = f"crosstransformer.layers.{i}", f"crosstransformer.layers_t.{i}"
        if i % 2 == 0:
            x, xt = self_layer(W, p, x, heads), self_layer(W, pt, xt, heads)
        else:
            old = x
            x = cross_layer(W, p, x, xt, heads)
            xt = cross_layer(W, pt, xt, old, heads)
        if trace is not None:
            trace[p], trace[pt] = x, xt
    x = x.reshape(B, T1, Fr, C).permute(0, 3, 2, 1)
    return x, xt.transpose(1, 2)


def spec(x, nfft=4096):
    hl = nfft // 4
    length = x.shape[-1]
    le = int(math.ceil(length / hl))
    pad = hl // 2 * 3
    xp = F.pad(x, (pad, pad + le * hl - length), mode="reflect")
    flat = xp.reshape(-1, xp.shape[-1])
    z = torch.stft(flat, nfft, hl, window=torch.hann_window(nfft, dtype=DT), win_length=nfft, normalized=True,
                   center=True, return_complex=True, pad_mode="reflect")
    z = z.view(*x.shape[:-1], z.shape[-2], z.shape[-1])[..., :-1, :]
    assert z.shape[-1] == le + 4
    return z[..., 2:2 + le]


def ispec(z, length, nfft=4096):
    hl = nfft // 4
    z = F.pad(z, (0, 0, 0, 1))
    z = F.pad(z, (2, 2))
    pad = hl // 2 * 3
    le = hl * int(math.ceil(length / hl)) + 2 * pad
    shape = z.shape
    flat = z.reshape(-1, shape[-2], shape[-1])
    x = torch.istft(flat, nfft, hl, window=torch.hann_window(nfft, dtype=DT), win_length=nfft, normalized=True,
                    length=le, center=True)
    x = x.view(*shape[:-2], -1)
    return x[..., pad:pad + length]


def forward(weights, mix, trace=None):
    """mix (B, 2, L) with L the training length; returns (B, 4, 2, L) float64."""
    W = weights if isinstance(weights, Weights) else Weights(weights)
    mix = T(mix)
    B, _, L = mix.shape
    z = spec(mix)
    mag = torch.view_as_real(z).permute(0, 1, 4, 2, 3).reshape(B, 4, z.shape[-2], z.shape[-1])
    mean = mag.mean(dim=(1, 2, 3), keepdim=True)
    std = mag.std(dim=(1, 2, 3), keepdim=True)
    x = (mag - mean) / (1e-5 + std)
    meant = mix.mean(dim=(1, 2), keepdim=True)
    stdt = mix.std(dim=(1, 2), keepdim=True)
    xt = (mix - meant) / (1e-5 + stdt)
    saved, saved_t, lengths_t = [], [], []
    for i in range(4):
        lengths_t.append(xt.shape[-1])
        xt = enc_time(W, i, xt)
        saved_t.append(xt)
        x = enc_freq(W, i, x)
        if i == 0:
            emb = (W["freq_emb.embedding.weight"] * 10.0).t()[None, :, :, None].expand_as(x)
            x = x + 0.2 * emb
        saved.append(x)
        if trace is not None:
            trace[f"tencoder.{i}"] = xt
            trace[f"encoder.{i}" if i else "encoder.0.post_emb"] = x
    b, c, f, t = x.shape
    x = F.conv1d(x.reshape(b, c, f * t), W["channel_upsampler.weight"], W["channel_upsampler.bias"]).view(b, -1, f, t)
    xt = F.conv1d(xt, W["channel_upsampler_t.weight"], W["channel_upsampler_t.bias"])
    x, xt = transformer(W, x, xt, trace=trace)
    x = F.conv1d(x.reshape(b, -1, f * t), W["channel_downsampler.weight"], W["channel_downsampler.bias"]).view(b, c, f, t)
    xt = F.conv1d(xt, W["channel_downsampler_t.weight"], W["channel_downsampler_t.bias"])
    for i in range(4):
        last = i == 3
        x = dec_freq(W, 3 - i, x, saved.pop(), last)
        xt = dec_time(W, 3 - i, xt, saved_t.pop(), lengths_t.pop(), last)
        if trace is not None:
            trace[f"decoder.{i}#0"], trace[f"tdecoder.{i}#0"] = x, xt
    S = 4
    Fq, Tn = x.shape[-2], x.shape[-1]
    x = x.view(B, S, -1, Fq, Tn) * std[:, None] + mean[:, None]
    zc = torch.view_as_complex(x.view(B, S, -1, 2, Fq, Tn).permute(0, 1, 2, 4, 5, 3).contiguous())
    wave = ispec(zc, L)
    xt = xt.view(B, S, -1, L) * stdt[:, None] + meant[:, None]
    return (xt + wave).numpy()
