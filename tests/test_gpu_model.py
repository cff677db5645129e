"""End-to-end parity of the HIP forward against the CPU oracle: per-stem SNR
>= 60 dB and per-named-activation max |err| <= 1e-3 (fp32), on seeded inputs
and random-init weights; plus the SegmentForward contract (two groups in
flight, batch independence) and the error paths the C-ABI must raise.
"""
import dataclasses
import json

import numpy as np
import pytest
import torch
from safetensors.numpy import save as st_save

from conftest import small_config, snr_db

pytestmark = pytest.mark.gpu

TRACED = ["x_normalized", "xt_normalized", "tencoder.0", "tencoder.3", "encoder.1", "encoder.3",
          "channel_upsampler", "crosstransformer.layers.0", "crosstransformer.layers_t.1",
          "crosstransformer.layers.4", "channel_downsampler", "decoder.0#0", "tdecoder.2#0", "decoder.3#0",
          "tdecoder.3#0", "model_out"]


@pytest.fixture(scope="module")
def small(dmx, oracle):
    cfg = small_config(dmx, 11025)
    weights = dmx.random_init(0, cfg)
    return cfg, weights, dmx.Runner(weights, cfg), oracle.Model(weights, cfg)


def per_stem_snr(ref, out):
    return [snr_db(ref[:, s], out[:, s]) for s in range(ref.shape[1])]


@pytest.mark.parametrize("precision", ["fp32", "fp32_mfma"])
def test_forward_matches_oracle_per_stem_and_per_activation(dmx, small, precision):
    """Both fp32 settings: the default (transformer linears on three bf16
    planes per operand) and fp32 MFMA for every contraction."""
    cfg, weights, runner, model = small
    if precision == "fp32_mfma":
        runner = dmx.Runner(weights, cfg, precision=dmx.PRECISION_FP32_MFMA)
    mix = dmx.signals.gaussian_segments(0, 2, cfg.training_length)
    ref_trace, gpu_trace = {}, {}
    wants = lambda name: name in TRACED
    ref = model.forward(mix, ref_trace, wants)
    runner.set_trace(wants, lambda n, a: gpu_trace.__setitem__(n, a))
    try:
        out = runner.forward(mix)
    finally:
        runner.set_trace(None, None)
    snrs = per_stem_snr(ref, out)
    assert min(snrs) >= 60.0, snrs
    for name in TRACED:
        assert name in gpu_trace and name in ref_trace, name
        a, b = ref_trace[name], gpu_trace[name]
        assert a.shape == b.shape, (name, a.shape, b.shape)
        err = float(np.max(np.abs(a - b)))
        assert err <= 1e-3 * max(1.0, float(np.max(np.abs(a)))), (name, err)


def test_shorter_input_is_padded_and_trimmed(dmx, small):
    cfg, weights, runner, model = small
    mix = dmx.signals.gaussian_segments(3, 1, 9000)
    ref = model.forward(mix)
    out = runner.forward(mix)
    assert out.shape == (1, 4, 2, 9000)
    assert min(per_stem_snr(ref, out)) >= 60.0


def test_batch_elements_are_independent(dmx, small):
    cfg, weights, runner, model = small
    mix = dmx.signals.gaussian_segments(1, 2, cfg.training_length)
    both = runner.forward(mix)
    one = runner.forward(mix[1:2])
    assert snr_db(one[0], both[1]) > 100.0  # core/tests/demucs_alignment.rs:231-261


def test_two_groups_in_flight(dmx, small):
    cfg, weights, runner, model = small
    a = dmx.signals.gaussian_segments(4, 1, cfg.training_length)
    b = dmx.signals.gaussian_segments(5, 2, cfg.training_length)
    pa = runner.start(a)
    pb = runner.start(b)  # queued before `a` is collected
    out_a, out_b = runner.collect(pa), runner.collect(pb)
    np.testing.assert_array_equal(out_a, runner.forward(a))
    np.testing.assert_array_equal(out_b, runner.forward(b))


def test_shape_errors_are_reported(dmx, small):
    cfg, weights, runner, model = small
    with pytest.raises(dmx.DmxError) as e:
        runner.forward(np.zeros((1, 2, cfg.training_length + 1), np.float32))
    assert e.value.kind == "Shape"
    with pytest.raises(dmx.DmxError) as e:
        runner.forward(np.zeros((1, 3, 100), np.float32))
    assert e.value.kind == "Shape"


def test_missing_and_misshapen_weights_are_reported(dmx, small):
    cfg, weights, runner, model = small
    w = dict(weights)
    del w["encoder.2.rewrite.bias"]
    with pytest.raises(dmx.DmxError) as e:
        dmx.Runner(w, cfg)
    assert e.value.kind == "MissingWeight"
    w = dict(weights)
    w["decoder.1.conv_tr.weight"] = np.zeros((1, 2, 3), np.float32)
    with pytest.raises(dmx.DmxError) as e:
        dmx.Runner(w, cfg)
    assert e.value.kind == "WeightShape"


@pytest.mark.parametrize("shifts,group,progress", [(0, 3, True), (1, 1, True), (2, 2, True), (0, 1, False),
                                                   (1, 3, False), (2, 2, False)])
def test_separation_matches_oracle(dmx, oracle, small, shifts, group, progress):
    """The device chunk loop (global norm, centred chunks, batched forwards,
    triangular OLA, shift view, denormalisation) against the oracle's
    `separate` on a 1.2 s mix with 0.25 s segments. Without a progress
    callback consecutive chunk groups run on alternating stream pairs."""
    cfg, weights, runner, model = small
    mix = dmx.signals.synthetic_mix(11, 1.2)
    opts = dmx.SeparateOptions(shifts=shifts, overlap=0.25, batch_chunks=group)
    ref = oracle.separate([model], mix[0], mix[1], 44100, opts)
    seen = []
    out = dmx.separate_runners([runner], mix[0], mix[1], 44100, opts, on_progress=seen.append if progress else None)
    for s in range(4):
        assert snr_db(ref[s], out[s]) >= 60.0, (s, snr_db(ref[s], out[s]))
    if progress:
        assert seen and seen[-1].done == seen[-1].total
        assert all(a.done <= b.done for a, b in zip(seen, seen[1:]))


@pytest.mark.parametrize("group", [1, 2])
def test_two_lane_schedule_matches_one_lane(dmx, small, group):
    """The same separation with one stream pair (a trace sink that records
    nothing keeps the whole run on the main stream) and with alternating
    pairs, the second pair's group starting when the first reaches its
    transformer: the stems agree to the f64 atomics' summation order (far
    tighter than the 60 dB parity gate), so no buffer is reused or read
    across the lanes too early."""
    cfg, weights, runner, model = small
    mix = dmx.signals.synthetic_mix(13, 1.6)
    opts = dmx.SeparateOptions(shifts=0, overlap=0.25, batch_chunks=group)
    runner.set_trace(lambda name: False, lambda name, a: None)
    try:
        one = dmx.separate_runners([runner], mix[0], mix[1], 44100, opts)
    finally:
        runner.set_trace(None, None)
    two = dmx.separate_runners([runner], mix[0], mix[1], 44100, opts)
    for s in range(4):
        assert snr_db(one[s], two[s]) >= 120.0, (s, snr_db(one[s], two[s]))


def test_bag_and_stem_selection_match_oracle(dmx, oracle):
    """A two-network bag with a non-identity weight matrix, then only one stem
    requested (StemSelection::Some): the networks that contribute nothing are
    skipped and the other stems are left untouched."""
    cfg = small_config(dmx, 11025)
    nets_w = [dmx.random_init(seed, cfg) for seed in (1, 2)]
    runners = [dmx.Runner(w, cfg) for w in nets_w]
    models = [oracle.Model(w, cfg) for w in nets_w]
    bag = np.array([[1.0, 0.0, 0.5, 0.0], [0.0, 1.0, 0.5, 1.0]], np.float32)
    mix = dmx.signals.synthetic_mix(12, 0.8)
    opts = dmx.SeparateOptions(shifts=0, batch_chunks=2)
    ref = oracle.separate(models, mix[0], mix[1], 44100, opts, bag_weights=bag)
    out = dmx.separate_runners(runners, mix[0], mix[1], 44100, opts, bag_weights=bag)
    for s in range(4):
        assert snr_db(ref[s], out[s]) >= 60.0, s
    wanted = [False, False, False, True]
    ref_v = oracle.separate(models, mix[0], mix[1], 44100, opts, bag_weights=bag, wanted=wanted)
    out_v = dmx.separate_runners(runners, mix[0], mix[1], 44100, opts, bag_weights=bag, wanted=wanted)
    assert snr_db(ref_v[3], out_v[3]) >= 60.0
    assert not out_v[:3].any()
    demucs = dmx.Demucs(runners, bag, dmx.LoadOptions(stems=dmx.StemSelection.some([dmx.StemId.VOCALS])))
    stems = demucs.separate_with_options(mix[0], mix[1], 44100, opts)
    assert [st.id for st in stems] == [dmx.StemId.VOCALS]
    assert snr_db(ref_v[3, 0], stems[0].left) >= 60.0


def test_sample_rate_mismatch_is_reported(dmx, small):
    cfg, weights, runner, model = small
    with pytest.raises(dmx.DmxError) as e:
        dmx.separate_runners([runner], np.zeros(5000, np.float32), np.zeros(5000, np.float32), 48000,
                             dmx.SeparateOptions())
    assert e.value.kind == "Shape"


def test_full_segment_forward_matches_oracle(dmx, oracle):
    """one 7.8 s segment, seed-0 weights, N(0, 0.1^2) input."""
    cfg = dmx.Config()
    weights = dmx.random_init(0, cfg)
    mix = dmx.signals.gaussian_segments(0, 1, cfg.training_length)
    out = dmx.Runner(weights, cfg).forward(mix)
    ref = oracle.Model(weights, cfg).forward(mix)
    snrs = per_stem_snr(ref, out)
    assert min(snrs) >= 60.0, snrs


def test_forward_matches_the_golden_fixture(dmx):
    """The HIP forward against the committed float64-torch fixture directly
    (no oracle in the loop): stems and sampled named activations."""
    from test_golden import check_fingerprints, golden, l4096_config
    g = golden("htdemucs_L4096_seed0.npz")
    cfg = l4096_config(dmx)
    runner = dmx.Runner(dmx.random_init(0, cfg), cfg)
    trace = {}
    runner.set_trace(None, lambda n, a: trace.__setitem__(n, a))
    try:
        out = runner.forward(g["mix"])
    finally:
        runner.set_trace(None, None)
    snrs = per_stem_snr(g["stems"], out)
    assert min(snrs) >= 60.0, snrs
    check_fingerprints(g, trace, 1e-3)


def _device_transformer(dmx, runner, x, xt):
    import torch
    b, d, f, t = x.shape
    dx, dxt = torch.from_numpy(x).cuda(), torch.from_numpy(xt).cuda()
    ox, oxt = torch.empty_like(dx), torch.empty_like(dxt)
    torch.cuda.synchronize()
    runner.crosstransformer_device(dx.data_ptr(), dxt.data_ptr(), b, f, t, xt.shape[-1], ox.data_ptr(), oxt.data_ptr())
    runner.synchronize()
    return ox.cpu().numpy(), oxt.cpu().numpy()


def test_crosstransformer_matches_the_golden_stack(dmx):
    """dmx_crosstransformer_device (config 2's entry point) on the fixture's
    4x6 + 12 tokens, Xavier-init seed 2."""
    from test_golden import golden
    g = golden("transformer_F4T6_seed2.npz")
    cfg = dmx.Config()
    runner = dmx.Runner(dmx.xavier_transformer_init(2, cfg), cfg)
    xo, xto = _device_transformer(dmx, runner, g["x"], g["xt"])
    assert snr_db(g["out"], xo) >= 60.0 and snr_db(g["out_t"], xto) >= 60.0


def test_crosstransformer_full_token_count_matches_oracle(dmx, oracle):
    """BASELINE config 2 at batch 1: 2688 frequency tokens (8 x 336) and 1344
    time tokens, N(0, 1) activations, Xavier-init transformer."""
    cfg = dmx.Config()
    w = dmx.xavier_transformer_init(2, cfg)
    r = np.random.default_rng(21)
    x = r.normal(size=(1, 512, 8, 336)).astype(np.float32)
    xt = r.normal(size=(1, 512, 1344)).astype(np.float32)
    xo, xto = _device_transformer(dmx, dmx.Runner(w, cfg), x, xt)
    ro, rto = oracle.Model(w, cfg).transformer(x, xt)
    assert snr_db(ro, xo) >= 60.0 and snr_db(rto, xto) >= 60.0
    assert float(np.abs(ro - xo).max()) <= 1e-3 * max(1.0, float(np.abs(ro).max()))


def test_bf16_forward_meets_the_40_db_gate(dmx, oracle):
    """BASELINE config 5's check on two of its segments: the bf16-MFMA runner
    (seed-7 weights, N(0, 0.1^2) input) against the fp32 oracle, per-stem
    SNR >= 40 dB; and it really is the bf16 path (below fp32 agreement)."""
    cfg = dmx.Config()
    w = dmx.random_init(7, cfg)
    mix = dmx.signals.gaussian_segments(7, 2, cfg.training_length)
    out = dmx.Runner(w, cfg, precision=dmx.PRECISION_BF16).forward(mix)
    ref = oracle.Model(w, cfg).forward(mix)
    snrs = per_stem_snr(ref, out)
    assert min(snrs) >= 40.0, snrs
    assert max(snrs) < 100.0, snrs


def test_bf16_separation_meets_the_40_db_gate(dmx, oracle, small):
    cfg, weights, _, model = small
    runner = dmx.Runner(weights, cfg, precision=dmx.PRECISION_BF16)
    mix = dmx.signals.synthetic_mix(13, 1.0)
    opts = dmx.SeparateOptions(shifts=1, overlap=0.25, batch_chunks=4)
    ref = oracle.separate([model], mix[0], mix[1], 44100, opts)
    out = dmx.separate_runners([runner], mix[0], mix[1], 44100, opts)
    for s in range(4):
        assert snr_db(ref[s], out[s]) >= 40.0, (s, snr_db(ref[s], out[s]))


@pytest.mark.parametrize("container", ["safetensors", "th"])
def test_a_checkpoint_file_loads_into_the_device_forward(dmx, oracle, small, tmp_path, container):
    """`Demucs.load(path)`: weights stored as F16 (as the published checkpoints
    are) come back widened to f32, the safetensors kwargs give the config, and
    the forward matches the oracle run on the same widened weights."""
    cfg, weights, _, _ = small
    w16 = {k: v.astype(np.float16) for k, v in weights.items()}
    if container == "safetensors":
        path = tmp_path / "net.safetensors"
        kwargs = dataclasses.asdict(cfg)
        kwargs["sources"] = list(dmx.Config.SOURCES)
        kwargs["cac"] = bool(kwargs["cac"])
        path.write_bytes(st_save(w16, metadata={"kwargs": json.dumps(kwargs)}))
        net = dmx.Demucs.load(str(path))
    else:
        path = tmp_path / "net.th"
        torch.save({"klass": None, "kwargs": {}, "state": {k: torch.from_numpy(v) for k, v in w16.items()}}, path)
        net = dmx.Demucs.load(path, config=cfg)
    assert net.runners[0].config == cfg
    mix = dmx.signals.gaussian_segments(4, 1, cfg.training_length)
    out = net.forward_segment(mix)
    ref = oracle.Model({k: v.astype(np.float32) for k, v in w16.items()}, cfg).forward(mix)
    snrs = per_stem_snr(ref, out)
    assert min(snrs) >= 60.0, snrs
