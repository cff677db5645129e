"""The BASELINE workloads at the sizes bench.py runs them, under parity or
property checks:

- config 1: one 7.8 s segment, per stem and per named activation;
- config 2: the cross-transformer stack at batch 8, one row against the
  oracle and every row against its own batch-1 run;
- config 3: the 60 s separation exactly as bench.py runs it (host samples in,
  8-chunk groups, two lanes) against the oracle's separation;
- config 4: the 180 s four-network bag with shifts=1, by the reference's bag
  properties (crates/demucs-core/tests/api_facade.rs:233-272);
- config 5: the bf16 forward at batch 32 against the fp32 oracle and against
  its own batch-1 runs (crates/demucs-core/tests/demucs_alignment.rs:231-261).

fp32 gates: per-stem SNR >= 60 dB, per-activation max |err| <= 1e-3 (relative
to max(1, max |ref|)); bf16: per-stem SNR >= 40 dB.
"""
import numpy as np
import pytest
import torch

from conftest import snr_db

pytestmark = pytest.mark.gpu

# Every named activation the forward records, from the first normalisation
# to the model output (names as in crates/demucs-core/src/demucs/host.rs:231-518).
TRACED_FULL = ["x_normalized", "xt_normalized"] + [f"encoder.{i}" for i in range(4)] + \
    [f"tencoder.{i}" for i in range(4)] + ["channel_upsampler", "channel_upsampler_t"] + \
    [f"crosstransformer.layers.{i}" for i in range(5)] + [f"crosstransformer.layers_t.{i}" for i in range(5)] + \
    ["channel_downsampler", "channel_downsampler_t"] + [f"decoder.{i}#0" for i in range(4)] + \
    [f"tdecoder.{i}#0" for i in range(4)] + [f"decoder.{i}#1" for i in range(4)] + \
    [f"tdecoder.{i}#1" for i in range(4)] + ["crosstransformer.in#0", "crosstransformer.in#1",
                                             "encoder.0.post_emb", "model_out"]


def per_stem_snr(ref, out):
    return [snr_db(ref[:, s], out[:, s]) for s in range(ref.shape[1])]


def test_config1_full_segment_per_stem_and_per_activation(dmx, oracle):
    """Config 1: seed-0 weights, one 7.8 s segment of N(0, 0.1^2) noise; every
    named activation both sides record is compared."""
    cfg = dmx.Config()
    weights = dmx.random_init(0, cfg)
    mix = dmx.signals.gaussian_segments(0, 1, cfg.training_length)
    wants = lambda name: name in TRACED_FULL
    ref_trace, gpu_trace = {}, {}
    ref = oracle.Model(weights, cfg).forward(mix, ref_trace, wants)
    runner = dmx.Runner(weights, cfg)
    runner.set_trace(wants, lambda n, a: gpu_trace.__setitem__(n, a))
    try:
        out = runner.forward(mix)
    finally:
        runner.set_trace(None, None)
    snrs = per_stem_snr(ref, out)
    assert min(snrs) >= 60.0, snrs
    compared = sorted(set(ref_trace) & set(gpu_trace))
    assert len(compared) >= 40, compared
    for name in compared:
        a, b = ref_trace[name], gpu_trace[name]
        assert a.shape == b.shape, (name, a.shape, b.shape)
        err = float(np.max(np.abs(a.astype(np.float64) - b)))
        assert err <= 1e-3 * max(1.0, float(np.max(np.abs(a)))), (name, err)


def _transformer(runner, x, xt):
    b, d, f, t = x.shape
    dx, dxt = torch.from_numpy(x).cuda(), torch.from_numpy(xt).cuda()
    ox, oxt = torch.empty_like(dx), torch.empty_like(dxt)
    torch.cuda.synchronize()
    runner.crosstransformer_device(dx.data_ptr(), dxt.data_ptr(), b, f, t, xt.shape[-1], ox.data_ptr(), oxt.data_ptr())
    runner.synchronize()
    return ox.cpu().numpy(), oxt.cpu().numpy()


def test_config2_transformer_batch8(dmx, oracle):
    """Config 2 at B = 8 (as bench.py times it): row 5 against the oracle's
    stack, and every row against the batch-1 run of its own input."""
    cfg = dmx.Config()
    w = dmx.xavier_transformer_init(0, cfg)
    runner = dmx.Runner(w, cfg)
    r = np.random.default_rng(8)
    x = r.normal(size=(8, 512, 8, 336)).astype(np.float32)
    xt = r.normal(size=(8, 512, 1344)).astype(np.float32)
    xo, xto = _transformer(runner, x, xt)
    ro, rto = oracle.Model(w, cfg).transformer(x[5:6], xt[5:6])
    assert snr_db(ro, xo[5:6]) >= 60.0 and snr_db(rto, xto[5:6]) >= 60.0
    assert float(np.abs(ro - xo[5:6]).max()) <= 1e-3 * max(1.0, float(np.abs(ro).max()))
    for i in range(8):
        so, sto = _transformer(runner, x[i:i + 1], xt[i:i + 1])
        assert snr_db(so, xo[i:i + 1]) > 100.0 and snr_db(sto, xto[i:i + 1]) > 100.0, i


def test_config3_separation_as_benchmarked(dmx, oracle):
    """Config 3 exactly as bench.py's `value` runs it: the 60 s seed-0 mix from
    host memory, 7.8 s segments at overlap 0.25 in groups of 8 (11 chunks: 8 +
    3, on the two lanes), shifts = 0, seed-0 weights."""
    cfg = dmx.Config()
    weights = dmx.random_init(0, cfg)
    mix = dmx.signals.synthetic_mix(0, 60.0)
    opts = dmx.SeparateOptions(shifts=0, overlap=0.25, batch_chunks=8)
    out = dmx.separate_runners([dmx.Runner(weights, cfg)], mix[0], mix[1], cfg.samplerate, opts)
    ref = oracle.separate([oracle.Model(weights, cfg)], mix[0], mix[1], cfg.samplerate, opts)
    assert out.shape == ref.shape == (4, 2, mix.shape[1])
    snrs = [snr_db(ref[s], out[s]) for s in range(4)]
    assert min(snrs) >= 60.0, snrs


def test_config4_bag_properties_at_full_size(dmx):
    """Config 4 (180 s, four seed-1..4 networks, identity bag, shifts = 1,
    groups of 8): with the identity matrix stem s of the bag is network s's
    own separation, and the vocals-only run (three networks pruned) gives the
    same vocals and leaves the other rows untouched."""
    cfg = dmx.Config()
    runners = [dmx.Runner(dmx.random_init(seed, cfg), cfg) for seed in (1, 2, 3, 4)]
    mix = dmx.signals.synthetic_mix(0, 180.0)
    opts = dmx.SeparateOptions(shifts=1, overlap=0.25, batch_chunks=8)
    bag = np.eye(4, dtype=np.float32)
    both = dmx.separate_runners(runners, mix[0], mix[1], cfg.samplerate, opts, bag_weights=bag)
    assert np.isfinite(both).all()
    for s in range(4):
        alone = dmx.separate_runners([runners[s]], mix[0], mix[1], cfg.samplerate, opts)
        assert snr_db(alone[s], both[s]) >= 120.0, (s, snr_db(alone[s], both[s]))
    vocals = dmx.separate_runners(runners, mix[0], mix[1], cfg.samplerate, opts, bag_weights=bag,
                                  wanted=[False, False, False, True])
    assert not vocals[:3].any()
    assert snr_db(both[3], vocals[3]) >= 120.0


def test_config5_bf16_batch32(dmx, oracle):
    """Config 5: the bf16-MFMA forward of 32 segments (seed-7 weights and
    input); segments 0 and 31 against the fp32 oracle, and three segments
    against their batch-1 bf16 runs."""
    cfg = dmx.Config()
    w = dmx.random_init(7, cfg)
    runner = dmx.Runner(w, cfg, precision=dmx.PRECISION_BF16)
    mix = dmx.signals.gaussian_segments(7, 32, cfg.training_length)
    out = runner.forward(mix)
    assert np.isfinite(out).all()
    model = oracle.Model(w, cfg)
    for i in (0, 31):
        snrs = per_stem_snr(model.forward(mix[i:i + 1]), out[i:i + 1])
        assert min(snrs) >= 40.0, (i, snrs)
    for i in (0, 13, 31):
        one = runner.forward(mix[i:i + 1])
        assert min(per_stem_snr(one, out[i:i + 1])) > 100.0, i
