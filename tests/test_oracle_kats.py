"""The reference's own known-answer tests, replayed against the CPU oracle.

Each test restates one `#[test]` of the reference with its hand-computed
expectation (inputs and expected outputs are data copied from those tests):
crates/demucs-core/src/demucs/ops.rs:1620-1777, crates/demucs-core/src/ops.rs:248-295,
crates/demucs-core/src/dsp/stft.rs:333-444, crates/demucs-core/src/demucs/config.rs:453-504,
crates/demucs-core/src/demucs/pipeline.rs:714-772.
"""
import math

import numpy as np
import pytest


def test_conv1d_matches_a_hand_written_correlation(oracle):  # ops.rs:1620-1630
    out = oracle.conv1d(np.array([[[1, 2, 3, 4]]]), np.array([[[1, 2]]]), np.array([0.5]), 1, 0, 1)
    assert out.shape == (1, 1, 3)
    np.testing.assert_allclose(out[0, 0], [1 + 4 + 0.5, 2 + 6 + 0.5, 3 + 8 + 0.5], atol=1e-6)


def test_conv1d_pads_with_zeros_and_respects_stride(oracle):  # ops.rs:1632-1642
    out = oracle.conv1d(np.array([[[1, 2, 3, 4, 5, 6]]]), np.ones((1, 1, 3)), np.zeros(1), 2, 1, 1)
    np.testing.assert_allclose(out[0, 0], [3, 9, 15], atol=1e-6)


def test_conv1d_dilation_spreads_the_taps(oracle):  # ops.rs:1644-1654
    out = oracle.conv1d(np.array([[[1, 2, 3, 4, 5]]]), np.array([[[1, 10]]]), np.zeros(1), 1, 2, 2)
    assert out.shape == (1, 1, 7)
    assert abs(out[0, 0, 0] - 10) < 1e-6
    assert abs(out[0, 0, 2] - 31) < 1e-6
    assert abs(out[0, 0, 6] - 5) < 1e-6


def test_conv_transpose1d_scatters_taps(oracle):  # ops.rs:1656-1667
    out = oracle.conv_transpose1d(np.array([[[1, 2]]]), np.array([[[1, 10]]]), np.zeros(1), 2)
    np.testing.assert_allclose(out[0, 0], [1, 10, 2, 20], atol=1e-6)


def test_conv2d_handles_a_two_dimensional_kernel(oracle):  # ops.rs:1669-1683
    x = np.arange(1, 10, dtype=np.float32).reshape(1, 1, 3, 3)
    out = oracle.conv2d(x, np.array([1, 0, 0, 0], np.float32).reshape(1, 1, 2, 2), np.zeros(1))
    assert out.shape == (1, 1, 2, 2)
    assert (out[0, 0, 0, 0], out[0, 0, 0, 1], out[0, 0, 1, 0]) == (1.0, 2.0, 4.0)


def test_group_norm_normalises_each_group_over_every_other_axis(oracle):  # ops.rs:1685-1699
    out = oracle.group_norm(np.array([[[1, 2], [3, 4]]]), 1, [1, 1], [0, 0])
    mean, var = 2.5, ((1 - 2.5) ** 2 + (2 - 2.5) ** 2 + (3 - 2.5) ** 2 + (4 - 2.5) ** 2) / 4
    inv = 1 / math.sqrt(var + 1e-5)
    assert abs(out[0, 0, 0] - (1 - mean) * inv) < 1e-5
    assert abs(out[0, 1, 1] - (4 - mean) * inv) < 1e-5


def test_group_norm_applies_the_affine_per_channel(oracle):  # ops.rs:1701-1711
    out = oracle.group_norm(np.array([[[0, 1], [0, 1]]]), 1, [2, 3], [1, -1])
    inv = 1 / math.sqrt(0.25 + 1e-5)
    normalised = (0 - 0.5) * inv
    assert abs(out[0, 0, 0] - (normalised * 2 + 1)) < 1e-5
    assert abs(out[0, 1, 0] - (normalised * 3 - 1)) < 1e-5
    assert abs(out[0, 0, 1] - (-normalised * 2 + 1)) < 1e-5


def test_group_norm_splits_channels_into_independent_groups(oracle):  # ops.rs:1713-1727
    out = oracle.group_norm(np.array([[[1], [2], [100], [200]]]), 2, [1, 1, 1, 1], [0, 0, 0, 0])
    assert abs(out[0, 0, 0] + out[0, 1, 0]) < 1e-5
    assert abs(out[0, 2, 0] + out[0, 3, 0]) < 1e-5
    assert abs(out[0, 3, 0] - out[0, 1, 0]) < 1e-4


def test_layer_norm_matches_a_hand_computed_row(oracle):  # ops.rs:1729-1738
    out = oracle.layer_norm(np.array([[1, 2, 3, 4]]), np.ones(4), np.zeros(4))
    inv = 1 / math.sqrt(1.25 + 1e-5)
    assert abs(out[0, 0] - (1 - 2.5) * inv) < 1e-5
    assert abs(out[0, 3] - (4 - 2.5) * inv) < 1e-5


def test_glu_gates_the_first_half_with_the_second(oracle):  # ops.rs:1740-1748
    out = oracle.glu(np.array([1, 1, 2, 2, 0, 0, 0, 0], np.float32).reshape(1, 4, 2))
    assert out.shape == (1, 2, 2)
    assert abs(out[0, 0, 0] - 0.5) < 1e-6
    assert abs(out[0, 1, 1] - 1.0) < 1e-6


def test_matmul_bt_matches_an_explicit_transpose_product(oracle):  # ops.rs:1750-1758
    a = np.array([[1, 2], [3, 4]], np.float32)
    b = np.array([[1, 0], [0, 1], [1, 1]], np.float32)
    out = oracle.sgemm(a, b.T)
    assert out.shape == (2, 3)
    assert abs(out[0, 0] - 1) < 1e-6 and abs(out[1, 2] - 7) < 1e-6


def test_attention_head_is_a_scaled_softmax_times_v(oracle):  # ops.rs:1760-1770
    out = oracle.attention_head(np.array([[1, 0]]), np.array([[1, 0], [0, 1]]), np.array([[2, 0], [0, 8]]), 1.0)
    a = math.e / (math.e + 1)
    assert abs(out[0, 0] - a * 2) < 1e-5
    assert abs(out[0, 1] - (1 - a) * 8) < 1e-5


def test_std_unbiased_matches_numpy_style_sample_deviation(oracle):  # ops.rs:1772-1777
    assert abs(oracle.std_unbiased(np.array([1, 2, 3, 4])) - math.sqrt(5 / 3)) < 1e-6


def test_linear_adds_bias_and_matches_manual_matmul(oracle):  # crates/demucs-core/src/ops.rs:248-257
    w = np.array([[1, 2], [3, 4]], np.float32)
    x = np.array([[1, 1], [2, 0]], np.float32)
    out = oracle.sgemm(x, w.T) + np.array([0.5, -0.5], np.float32)
    assert abs(out[0, 0] - 3.5) < 1e-6 and abs(out[1, 1] - 5.5) < 1e-6


def test_gelu_matches_torch_exact_gelu(oracle):  # crates/demucs-core/src/ops.rs:276-287
    g = oracle.lib().oracle_gelu_scalar
    assert abs(g(0.0)) < 1e-7
    assert abs(g(1.0) - 0.84134471) < 1e-5
    assert abs(g(-1.0) - -0.15865529) < 1e-5
    assert abs(g(2.0) - 1.95449996) < 1e-5
    assert abs(g(-3.0) - -0.00404987) < 1e-6
    assert g(20.0) > 19.9
    assert abs(g(-20.0)) < 1e-6


def test_softmax_sums_to_one_and_handles_large_offsets(oracle):  # crates/demucs-core/src/ops.rs:289-295
    # attention_head's softmax with identical scores over v = identity rows.
    q = np.array([[1.0, 0.0, 0.0]], np.float32)
    k = np.array([[1000.0, 0.0, 0.0]] * 3, np.float32)
    v = np.eye(3, dtype=np.float32)
    out = oracle.attention_head(q, k, v, 1.0)
    assert abs(out.sum() - 1.0) < 1e-6
    assert abs(out[0, 0] - 1 / 3) < 1e-6


# ---- dsp/stft.rs tests ----

def test_hann_window_matches_the_periodic_definition(oracle):  # stft.rs:333-340
    np.testing.assert_allclose(oracle.hann_window(4), [0.0, 0.5, 1.0, 0.5], atol=1e-7)


def test_reflect_padding_mirrors_without_repeating_the_edge(oracle):  # stft.rs:342-346
    np.testing.assert_array_equal(oracle.pad1d_reflect(np.array([1, 2, 3, 4]), 3, 3),
                                  [4, 3, 2, 1, 2, 3, 4, 3, 2, 1])


def test_frame_count_follows_center_padding(oracle):  # stft.rs:348-354
    assert oracle.stft(np.zeros((1, 26460)), 2048, 441).shape[2] == 61
    assert oracle.stft(np.zeros((1, 441 * 60)), 2048, 441).shape[2] == 61


def test_a_single_bin_sinusoid_lands_in_the_expected_bin(oracle):  # stft.rs:356-371
    sig = np.sin(2 * np.pi * np.arange(256) / 8.0).astype(np.float32)[None]
    spec = oracle.stft(sig, 64, 16)
    assert int(np.argmax(np.abs(spec[0, :, 4]))) == 8


def test_forward_then_inverse_reconstructs_the_signal_interior(oracle):  # stft.rs:373-396
    t = np.arange(2048, dtype=np.float32)
    sig = (np.sin(t * 0.013) * 0.7 + np.cos(t * 0.11) * 0.3).astype(np.float32)[None]
    rebuilt = oracle.istft(oracle.stft(sig, 256, 64), 256, 64)
    assert rebuilt.shape == (1, 2048)
    assert np.max(np.abs(rebuilt[0, 300:-300] - sig[0, 300:-300])) < 1e-4


def test_normalized_forward_and_inverse_round_trip(oracle):  # stft.rs:398-421
    sig = np.sin(np.arange(1024, dtype=np.float32) * 0.037)[None]
    spec = oracle.stft(sig, 256, 64, normalized=True)
    raw = oracle.stft(sig, 256, 64)
    assert abs(abs(raw[0, 8, 4]) / abs(spec[0, 8, 4]) - 16.0) < 1e-2
    rebuilt = oracle.istft(spec, 256, 64, normalized=True, length=1024)
    assert np.max(np.abs(rebuilt[0, 200:-200] - sig[0, 200:-200])) < 1e-4


def test_inverse_length_matches_hop_times_frames_when_length_is_none(oracle):  # stft.rs:423-429
    assert oracle.istft(np.zeros((2, 1025, 5), np.complex64), 2048, 441).shape == (2, 441 * 4)


def test_explicit_length_is_honoured(oracle):  # stft.rs:431-437
    assert oracle.istft(np.zeros((1, 1025, 5), np.complex64), 2048, 441, length=1000).shape == (1, 1000)


def test_reflect_padding_rejects_inputs_shorter_than_the_pad(oracle):  # stft.rs:439-444
    with pytest.raises(oracle.OracleError):
        oracle.stft(np.zeros((1, 100)), 2048, 441)


# ---- config.rs tests ----

def test_the_layer_table_and_training_length(dmx):  # config.rs:453-504
    cfg = dmx.Config()
    assert cfg.training_length == 343980
    assert cfg.hop_length == 1024
    shapes = dmx.weight_shapes(cfg)
    enc = [shapes[f"encoder.{i}.conv.weight"] for i in range(4)]
    assert [(s[1], s[0]) for s in enc] == [(4, 48), (48, 96), (96, 192), (192, 384)]
    tenc = [shapes[f"tencoder.{i}.conv.weight"] for i in range(4)]
    assert [(s[1], s[0]) for s in tenc] == [(2, 48), (48, 96), (96, 192), (192, 384)]
    # execution order (innermost first) is construction index 3, 2, 1, 0
    dec = [shapes[f"decoder.{i}.conv_tr.weight"] for i in (3, 2, 1, 0)]
    assert [(s[0], s[1]) for s in dec] == [(384, 192), (192, 96), (96, 48), (48, 16)]
    tdec = [shapes[f"tdecoder.{i}.conv_tr.weight"] for i in (3, 2, 1, 0)]
    assert [(s[0], s[1]) for s in tdec] == [(384, 192), (192, 96), (96, 48), (48, 8)]
    assert shapes["freq_emb.embedding.weight"] == (512, 48)
    assert shapes["crosstransformer.layers.0.linear1.weight"] == (2048, 512)


# ---- pipeline.rs tests ----

def test_the_transition_window_rises_then_falls(oracle):  # pipeline.rs:714-721
    w = oracle.transition_weight(8, 1.0)
    assert len(w) == 8 and abs(w[3] - 1.0) < 1e-6
    assert w[0] < w[1] < w[2] and w[7] < w[6] < w[5]


def test_the_shift_rng_stays_in_range(oracle):  # pipeline.rs:765-772
    vals = oracle.shift_rng(7, 22050, 1000)
    assert vals.min() >= 0 and vals.max() <= 22050


def test_normalisation_round_trips(oracle):  # pipeline.rs:752-763
    wav = np.array([[[0.5, -0.25, 1.0, 0.0]], [[0.5, -0.25, 1.0, 0.0]]], np.float32)
    m, s = oracle.scan_norm(wav)
    back = ((wav - m) / s) * s + m
    np.testing.assert_allclose(back, wav, atol=1e-5)


def test_a_centred_chunk_takes_context_from_both_sides(oracle):  # pipeline.rs:723-732, mix.rs:552-585
    # TensorChunk.padded: a chunk of `len` samples at `offset` padded to `seg`
    # starts at offset - (seg - len) // 2 and takes real context on both sides.
    mix = np.arange(10, dtype=np.float32).reshape(1, 1, 10)
    chunks = []
    oracle.split_pass(mix, 8, 0.5, 1.0, 0, 0, 1, 1, lambda x: chunks.append(x.copy()) or x[:, None])
    assert len(chunks) == 3  # offsets 0, 4, 8 (stride 4)
    np.testing.assert_array_equal(chunks[0][0, 0], [0, 1, 2, 3, 4, 5, 6, 7])
    np.testing.assert_array_equal(chunks[1][0, 0], [3, 4, 5, 6, 7, 8, 9, 0])  # len 6 -> start 3
    np.testing.assert_array_equal(chunks[2][0, 0], [5, 6, 7, 8, 9, 0, 0, 0])  # len 2 -> start 5


def test_a_chunk_at_the_start_is_zero_padded_on_the_left(oracle):  # pipeline.rs:734-742
    # padded_chunk(mix, 0, 3, 7) == [0, 0, 0, 1, 2, 3, 4]: a 3-sample tail chunk padded to 7.
    mix = np.arange(3, dtype=np.float32).reshape(1, 1, 3)
    chunks = []
    oracle.split_pass(mix, 7, 0.0, 1.0, 0, 0, 1, 1, lambda x: chunks.append(x.copy()) or x[:, None])
    np.testing.assert_array_equal(chunks[0][0, 0], [0, 0, 0, 1, 2, 0, 0])


def test_shift_rng_matches_the_closed_form_lcg(oracle):  # pipeline.rs:136-151
    state = (0x5EED1234 * 6364136223846793005 + 1) % 2 ** 64
    expect = []
    for _ in range(5):
        state = (state * 6364136223846793005 + 1442695040888963407) % 2 ** 64
        expect.append((state >> 33) % 22051)
    np.testing.assert_array_equal(oracle.shift_rng(0x5EED1234, 22050, 5), expect)
