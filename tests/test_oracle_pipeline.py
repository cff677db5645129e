"""Chunking / overlap-add / shift / bag invariants of the oracle's separation
loop, with stand-in forwards (the reference's `IdForward` pattern,
crates/demucs-core/src/demucs/streaming.rs:657-926, core/tests/streaming_ola.rs:109-233).
"""
import numpy as np
import pytest

from conftest import snr_db


def identity_forward(chunk):
    """Every source gets the chunk itself: the OLA must give the mix back."""
    return np.repeat(chunk[:, None], 4, axis=1)


def scaled_forward(chunk):
    """Source s gets (s + 1) * chunk (a linear, source-dependent stand-in)."""
    return np.stack([chunk * (s + 1) for s in range(4)], axis=1)


@pytest.mark.parametrize("length,seg,group", [(1000, 160, 1), (1000, 160, 3), (159, 160, 1), (161, 160, 2),
                                              (4000, 1000, 8)])
def test_identity_forward_reconstructs_the_normalised_mix(oracle, length, seg, group):
    mix = np.random.default_rng(length).normal(size=(1, 2, length)).astype(np.float32)
    out = oracle.split_pass(mix, seg, 0.25, 1.0, 0, 0, group, 4, identity_forward)
    for s in range(4):
        np.testing.assert_allclose(out[0, s], mix[0], rtol=1e-5, atol=1e-6)


def test_grouping_is_a_scheduling_change_only(oracle):  # pipeline.rs:774-839
    mix = np.random.default_rng(1).normal(size=(1, 2, 2500)).astype(np.float32)
    one = oracle.split_pass(mix, 400, 0.25, 1.0, 0, 0, 1, 4, scaled_forward)
    three = oracle.split_pass(mix, 400, 0.25, 1.0, 0, 0, 3, 4, scaled_forward)
    np.testing.assert_array_equal(one, three)


def test_chunk_count_is_ceil_length_over_stride(oracle):  # streaming.rs:87-94
    calls = []
    mix = np.zeros((1, 2, 687960), np.float32)
    oracle.split_pass(mix, 343980, 0.25, 1.0, 0, 0, 1, 4, lambda c: calls.append(1) or identity_forward(c))
    assert len(calls) == 3  # num_chunks_for(687960, 343980, 257985) == 3


@pytest.mark.parametrize("shifts", [0, 1, 2])
def test_separate_with_identity_forward_returns_the_mix(dmx, oracle, shifts):
    """Global normalisation, chunking, OLA, shift view + trim and the final
    denormalisation compose to the identity."""
    rng = np.random.default_rng(shifts)
    left, right = (rng.normal(size=30000) * 0.3).astype(np.float32), (rng.normal(size=30000) * 0.3).astype(np.float32)
    opts = dmx.SeparateOptions(shifts=shifts, overlap=0.25, segment=4410 / 44100, batch_chunks=2)
    out = oracle.separate([], left, right, 44100, opts, forward=identity_forward)
    for s in range(4):
        assert snr_db(left, out[s, 0]) > 110 and snr_db(right, out[s, 1]) > 110


def test_a_linear_forward_commutes_with_the_overlap_add(dmx, oracle):
    """Scaling a source inside the forward scales the normalised stem: the OLA,
    trim and denormalisation are linear in the forward's output."""
    rng = np.random.default_rng(3)
    left, right = rng.normal(size=9000).astype(np.float32), rng.normal(size=9000).astype(np.float32)
    opts = dmx.SeparateOptions(shifts=0, segment=2205 / 44100)
    single = oracle.separate([], left, right, 44100, opts, forward=scaled_forward)
    ident = oracle.separate([], left, right, 44100, opts, forward=identity_forward)
    # stem s of the scaled forward is (s + 1) times the identity's, minus the
    # (s + 1 - 1) * mean offset the denormalisation adds once.
    m, sd = oracle.scan_norm(np.stack([left, right])[None])
    for s in range(4):
        expect = (ident[s] - m) * (s + 1) + m
        assert snr_db(expect, single[s]) > 100


def test_a_bag_is_the_weight_normalised_sum_of_its_networks(dmx, oracle):
    """BagCombine (crates/demucs-core/src/api.rs:319-371, :883-971): stem s of
    a bag is sum_n w[n][s] * y_n[s] / sum_n w[n][s]; with a one-hot matrix it
    is exactly one network's separation (core/tests/api_facade.rs:233-272)."""
    from conftest import small_config
    cfg = small_config(dmx, 11025)
    models = [oracle.Model(dmx.random_init(seed, cfg), cfg) for seed in (1, 2)]
    mix = dmx.signals.synthetic_mix(5, 0.7)
    opts = dmx.SeparateOptions(shifts=0, batch_chunks=2)
    single = [oracle.separate([m], mix[0], mix[1], 44100, opts) for m in models]
    bag = np.array([[1.0, 0.25, 0.0, 2.0], [0.0, 0.75, 1.0, 1.0]], np.float32)
    both = oracle.separate(models, mix[0], mix[1], 44100, opts, bag_weights=bag)
    for s in range(4):
        expect = (bag[0, s] * single[0][s].astype(np.float64) + bag[1, s] * single[1][s]) / bag[:, s].sum()
        assert snr_db(expect, both[s]) > 100.0, s
    np.testing.assert_array_equal(both[0], single[0][0])
    np.testing.assert_array_equal(both[2], single[1][2])


def _triangle(seg, power):
    """The weight of crates/demucs-core/src/demucs/pipeline.rs:117-131 written
    out here: 1..=seg/2 rising, then seg - seg/2 down to 1, divided by its
    maximum, raised to `power`."""
    half = seg // 2
    w = np.concatenate([np.arange(1, half + 1), np.arange(seg - half, 0, -1)]).astype(np.float64)
    return (w / max(w.max(), 1.0)) ** power


@pytest.mark.parametrize("length,seg,power,group", [(1000, 160, 1.0, 1), (1000, 161, 1.0, 2), (777, 100, 2.0, 3),
                                                    (5000, 1000, 0.5, 4)])
def test_overlap_add_weights_chunks_by_the_triangle(oracle, length, seg, power, group):
    """A stand-in forward that answers chunk i with the constant i + 1: the
    overlap-add at sample t must be sum_i w(t - s_i) (i + 1) / sum_i w(t - s_i)
    over the chunks covering t (splice_group, pipeline.rs:660-699: a chunk of
    length n uses weights [0, n) and the centre-trimmed output). A wrong
    weight shape, offset or normalisation changes the ratio."""
    calls = []

    def index_forward(chunk):
        first = sum(calls)  # chunks answered by earlier groups
        calls.append(chunk.shape[0])
        out = np.empty((chunk.shape[0], 4) + chunk.shape[1:], np.float32)
        for j in range(chunk.shape[0]):
            out[j] = first + j + 1
        return out

    mix = np.zeros((1, 2, length), np.float32)
    out = oracle.split_pass(mix, seg, 0.25, power, 0, 0, group, 4, index_forward)
    stride = int(0.75 * seg)
    starts = list(range(0, length, stride))
    assert sum(calls) == len(starts)
    w = _triangle(seg, power)
    num = np.zeros(length)
    den = np.zeros(length)
    for i, s0 in enumerate(starts):
        n = min(length - s0, seg)
        num[s0:s0 + n] += w[:n] * (i + 1)
        den[s0:s0 + n] += w[:n]
    expect = num / den
    for s in range(4):
        for c in range(2):
            np.testing.assert_allclose(out[0, s, c], expect, rtol=2e-6)
