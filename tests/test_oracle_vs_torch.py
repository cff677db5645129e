"""Pins the CPU oracle against independent float64 PyTorch at small shapes.

Each reference host op documents the PyTorch call it mirrors
(crates/demucs-core/src/demucs/ops.rs:1-5); torch.nn.functional / torch.stft in
float64 is therefore an independent check of the oracle's restatement. The
model-level test compares the oracle's whole forward with a float64 torch
composition written from the upstream model's semantics (tests/torch_htdemucs.py).
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from conftest import rms_relative_error, small_config, snr_db

torch.set_num_threads(min(8, torch.get_num_threads()))


def t64(a):
    return torch.as_tensor(np.asarray(a, np.float64))


def rng(seed):
    return np.random.default_rng(seed)


@pytest.mark.parametrize("shape,stride,pad,dil", [((1, 4, 40, 7, 48, 8, 1), (4, 1), (2, 0), (1, 1)),
                                                  ((2, 6, 9, 11, 5, 3, 3), (1, 1), (1, 1), (1, 1)),
                                                  ((1, 3, 1, 50, 4, 1, 3), (1, 1), (0, 2), (1, 2)),
                                                  ((1, 2, 1, 64, 8, 1, 8), (1, 4), (0, 2), (1, 1))])
def test_conv2d(oracle, shape, stride, pad, dil):
    b, ic, h, w, oc, kh, kw = shape
    r = rng(sum(shape))
    x = r.normal(size=(b, ic, h, w)).astype(np.float32)
    wt = r.normal(size=(oc, ic, kh, kw)).astype(np.float32)
    bias = r.normal(size=oc).astype(np.float32)
    ref = F.conv2d(t64(x), t64(wt), t64(bias), stride=stride, padding=pad, dilation=dil).numpy()
    assert rms_relative_error(ref, oracle.conv2d(x, wt, bias, stride, pad, dil)) < 1e-6


@pytest.mark.parametrize("b,ic,h,w,oc,kh,kw,sh,sw", [(1, 5, 6, 3, 4, 8, 1, 4, 1), (2, 3, 1, 20, 2, 1, 8, 1, 4)])
def test_conv_transpose2d(oracle, b, ic, h, w, oc, kh, kw, sh, sw):
    r = rng(h * w)
    x = r.normal(size=(b, ic, h, w)).astype(np.float32)
    wt = r.normal(size=(ic, oc, kh, kw)).astype(np.float32)
    bias = r.normal(size=oc).astype(np.float32)
    ref = F.conv_transpose2d(t64(x), t64(wt), t64(bias), stride=(sh, sw)).numpy()
    assert rms_relative_error(ref, oracle.conv_transpose2d(x, wt, bias, (sh, sw))) < 1e-6


@pytest.mark.parametrize("groups", [1, 2, 4])
def test_group_norm(oracle, groups):
    r = rng(groups)
    x = (r.normal(size=(3, 8, 57)) * 3 + 1).astype(np.float32)
    w, b = r.normal(size=8).astype(np.float32), r.normal(size=8).astype(np.float32)
    ref = F.group_norm(t64(x), groups, t64(w), t64(b), eps=1e-5).numpy()
    assert rms_relative_error(ref, oracle.group_norm(x, groups, w, b)) < 1e-6


def test_group_norm_glu(oracle):
    r = rng(11)
    x = r.normal(size=(2, 12, 31)).astype(np.float32)
    w, b = r.normal(size=12).astype(np.float32), r.normal(size=12).astype(np.float32)
    ref = F.glu(F.group_norm(t64(x), 1, t64(w), t64(b), eps=1e-5), dim=1).numpy()
    assert rms_relative_error(ref, oracle.group_norm_glu(x, 1, w, b)) < 1e-6


def test_layer_norm(oracle):
    r = rng(3)
    x = (r.normal(size=(17, 512)) * 2 - 0.5).astype(np.float32)
    w, b = r.normal(size=512).astype(np.float32), r.normal(size=512).astype(np.float32)
    ref = F.layer_norm(t64(x), (512,), t64(w), t64(b), eps=1e-5).numpy()
    assert rms_relative_error(ref, oracle.layer_norm(x, w, b)) < 1e-6


def test_glu_and_gelu(oracle):
    x = np.linspace(-9, 9, 4 * 50, dtype=np.float32).reshape(1, 4, 50)
    assert rms_relative_error(F.glu(t64(x), dim=1).numpy(), oracle.glu(x)) < 1e-6
    # exact (erf) GELU; the reference's rational erfc is accurate to ~1.2e-7 relative
    np.testing.assert_allclose(oracle.gelu(x), F.gelu(t64(x)).numpy(), rtol=1e-6, atol=1e-7)


def test_multi_head_attention(oracle):
    r = rng(5)
    b, nq, nk, dim, heads = 2, 9, 13, 128, 2
    q, k = r.normal(size=(b, nq, dim)).astype(np.float32), r.normal(size=(b, nk, dim)).astype(np.float32)
    ws = [r.normal(size=(dim, dim)).astype(np.float32) * 0.1 for _ in range(4)]
    bs = [r.normal(size=dim).astype(np.float32) * 0.1 for _ in range(4)]
    mha = torch.nn.MultiheadAttention(dim, heads, batch_first=True).double()
    with torch.no_grad():
        mha.in_proj_weight.copy_(t64(np.concatenate(ws[:3])))
        mha.in_proj_bias.copy_(t64(np.concatenate(bs[:3])))
        mha.out_proj.weight.copy_(t64(ws[3]))
        mha.out_proj.bias.copy_(t64(bs[3]))
        ref = mha(t64(q), t64(k), t64(k), need_weights=False)[0].numpy()
    out = oracle.multi_head_attention(q, k, heads, ws[0], bs[0], ws[1], bs[1], ws[2], bs[2], ws[3], bs[3])
    assert rms_relative_error(ref, out) < 1e-6


def test_fft_matches_the_dft_definition(oracle):
    x = rng(7).normal(size=64) + 1j * rng(8).normal(size=64)
    x = x.astype(np.complex64)
    np.testing.assert_allclose(oracle.fft(x), np.fft.fft(x.astype(np.complex128)), atol=1e-9 * 64)
    np.testing.assert_allclose(oracle.fft(x, inverse=True), np.fft.ifft(x.astype(np.complex128)) * 64, atol=1e-9 * 64)
    y = rng(9).normal(size=48).astype(np.float32)  # non power of two: direct DFT
    np.testing.assert_allclose(oracle.fft(y), np.fft.fft(y.astype(np.float64)), atol=1e-9 * 48)


@pytest.mark.parametrize("n_fft,hop,normalized", [(4096, 1024, True), (256, 64, False)])
def test_stft_and_istft(oracle, n_fft, hop, normalized):
    x = rng(n_fft).normal(size=(2, 9000)).astype(np.float32)
    win = torch.hann_window(n_fft, dtype=torch.float64)
    ref = torch.stft(t64(x), n_fft, hop, window=win, win_length=n_fft, normalized=normalized, center=True,
                     return_complex=True, pad_mode="reflect").numpy()
    spec = oracle.stft(x, n_fft, hop, normalized)
    assert snr_db(np.abs(ref), np.abs(spec)) > 120 and snr_db(ref.real, spec.real) > 120
    back_ref = torch.istft(torch.as_tensor(ref), n_fft, hop, window=win, win_length=n_fft, normalized=normalized,
                           length=9000, center=True).numpy()
    back = oracle.istft(ref.astype(np.complex64), n_fft, hop, normalized, length=9000)
    assert snr_db(back_ref, back) > 120


def test_spec_and_ispec_framing(oracle):
    import torch_htdemucs as th
    mix = rng(1).normal(0, 0.1, (2, 2, 11025)).astype(np.float32)
    z = th.spec(t64(mix))
    ref = torch.view_as_real(z).permute(0, 1, 4, 2, 3).reshape(2, 4, 2048, -1).numpy()
    out = oracle.spec_cac(mix)
    assert out.shape == ref.shape == (2, 4, 2048, 11)
    assert snr_db(ref, out) > 120
    xs = rng(2).normal(size=(1, 16, 2048, 11)).astype(np.float32)
    zc = torch.view_as_complex(t64(xs).view(1, 4, 2, 2, 2048, 11).permute(0, 1, 2, 4, 5, 3).contiguous())
    wave_ref = th.ispec(zc, 11025).numpy()
    assert snr_db(wave_ref, oracle.ispec_cac(xs, 4, 11025)) > 120


def test_positional_embeddings(oracle):
    import torch_htdemucs as th
    p2 = th.sin_2d(512, 8, 21).permute(0, 3, 2, 1).reshape(21 * 8, 512).numpy()
    np.testing.assert_allclose(oracle.positions_2d(512, 8, 21), p2, atol=2e-5)
    np.testing.assert_allclose(oracle.positions_1d(37, 512), th.sin_1d(37, 512).numpy(), atol=2e-5)


def test_full_model_matches_an_independent_torch_composition(dmx, oracle):
    """The whole forward (0.25 s segment of the real architecture, seed-0
    weights), oracle (f32) against a float64 torch composition."""
    import torch_htdemucs as th
    cfg = small_config(dmx, 11025)
    weights = dmx.random_init(0, cfg)
    mix = dmx.signals.gaussian_segments(0, 2, cfg.training_length)
    trace = {}
    out = oracle.Model(weights, cfg).forward(mix, trace)
    ttrace = {}
    ref = th.forward(weights, mix, ttrace)
    for s in range(4):
        assert snr_db(ref[:, s], out[:, s]) > 80.0, s
    for name in ["tencoder.0", "tencoder.3", "encoder.0.post_emb", "encoder.3", "crosstransformer.layers.1",
                 "crosstransformer.layers_t.3", "crosstransformer.layers.4", "decoder.0#0", "tdecoder.3#0"]:
        a = ttrace[name].numpy()
        assert snr_db(a, trace[name]) > 80.0, name


def test_transformer_stack_matches_torch(dmx, oracle):
    """BASELINE config 2's structure (5 layers alternating self / cross, 2-D and
    1-D embeddings) at a reduced token count, Xavier-init weights."""
    import torch_htdemucs as th
    cfg = dmx.Config()
    weights = dmx.xavier_transformer_init(2, cfg)
    r = rng(4)
    x = r.normal(size=(1, 512, 8, 12)).astype(np.float32)
    xt = r.normal(size=(1, 512, 48)).astype(np.float32)
    xo, xto = oracle.Model(weights, cfg).transformer(x, xt)
    W = th.Weights(weights)
    rx, rxt = th.transformer(W, t64(x), t64(xt))
    assert snr_db(rx.numpy(), xo) > 90 and snr_db(rxt.numpy(), xto) > 90


def test_weight_inventory_matches_the_reference_parameter_count(dmx):
    # 41,984,456 parameters for the htdemucs architecture (the count of weights.rs's
    # tensors, computed from the layer table).
    assert dmx.weights.parameter_count(dmx.random_init(0)) == 41984456
