"""The oracle against the committed golden fixtures in tests/golden/ (written
by make_golden.py from the float64 torch composition, tests/torch_htdemucs.py):
the seeded weight recipe, the full forward with named-activation
fingerprints, and the cross-transformer stack."""
from pathlib import Path

import numpy as np

from conftest import snr_db

GOLDEN = Path(__file__).resolve().parent / "golden"


def golden(name):
    return np.load(GOLDEN / name)  # plain arrays only (allow_pickle=False)


def key(name):
    return name.replace(".", "_").replace("#", "_")


def l4096_config(dmx):
    cfg = dmx.Config()
    cfg.segment = 4096 / cfg.samplerate
    assert cfg.training_length == 4096
    return cfg


def check_weight_sums(g, weights):
    names = [str(n) for n in g["weights_names"]]
    assert sorted(weights) == names
    sums = np.array([weights[n].astype(np.float64).sum() for n in names])
    np.testing.assert_allclose(sums, g["weights_sum"], rtol=1e-12, atol=1e-9)


def check_fingerprints(g, trace, tol):
    for name in [str(n) for n in g["traced"]]:
        a = np.asarray(trace[name], np.float64)
        k = key(name)
        assert tuple(a.shape) == tuple(g[f"act_{k}_shape"]), name
        rms = float(np.sqrt(g[f"act_{k}_sumsq"] / a.size))
        err = np.abs(a.ravel()[g[f"act_{k}_index"]] - g[f"act_{k}_sample"])
        assert float(err.max()) <= tol * max(1.0, rms), (name, float(err.max()), rms)
        assert abs(float((a * a).sum()) - float(g[f"act_{k}_sumsq"])) <= 1e-4 * float(g[f"act_{k}_sumsq"]), name


def test_the_weight_recipe_is_unchanged(dmx):
    check_weight_sums(golden("htdemucs_L4096_seed0.npz"), dmx.random_init(0, l4096_config(dmx)))
    g = golden("transformer_F4T6_seed2.npz")
    w = dmx.xavier_transformer_init(2, dmx.Config())
    check_weight_sums(g, {k: v for k, v in w.items() if k.startswith("crosstransformer.")})


def test_oracle_forward_matches_the_golden_stems_and_activations(dmx, oracle):
    g = golden("htdemucs_L4096_seed0.npz")
    cfg = l4096_config(dmx)
    np.testing.assert_array_equal(g["mix"], dmx.signals.gaussian_segments(0, 1, 4096))
    trace = {}
    out = oracle.Model(dmx.random_init(0, cfg), cfg).forward(g["mix"], trace)
    for s in range(4):
        assert snr_db(g["stems"][:, s], out[:, s]) > 80.0, s
    check_fingerprints(g, trace, 1e-4)


def test_oracle_transformer_matches_the_golden_stack(dmx, oracle):
    g = golden("transformer_F4T6_seed2.npz")
    cfg = dmx.Config()
    xo, xto = oracle.Model(dmx.xavier_transformer_init(2, cfg), cfg).transformer(g["x"], g["xt"])
    assert snr_db(g["out"], xo) > 90.0
    assert snr_db(g["out_t"], xto) > 90.0
