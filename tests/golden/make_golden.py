"""Writes the committed golden fixtures of this directory.

Both fixtures come from tests/torch_htdemucs.py, the float64 torch composition
of HTDemucs v4 written from the upstream PyTorch semantics, on inputs and
weights made by the package's own seeded generators (SplitMix64 streams, so
the weights are reproducible bit for bit without storing them; their
checksums are stored to catch a drifting recipe).

  htdemucs_L4096_seed0.npz   full forward, real architecture, 4096-sample
                             segment (4 STFT frames), random-init seed 0,
                             N(0, 0.1^2) stereo input: mix, stems and a
                             fingerprint (shape, sum, sum of squares, 64
                             strided samples) of each named activation.
  transformer_F4T6_seed2.npz the 5-layer cross-transformer (config 2's
                             structure) on 4x6 frequency tokens and 12 time
                             tokens, Xavier-init seed 2: inputs and outputs.

Run from the repository root:  python tests/golden/make_golden.py
"""
import importlib.util
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(HERE.parent))

TRACED = ["tencoder.0", "tencoder.3", "encoder.0.post_emb", "encoder.3", "crosstransformer.layers.1",
          "crosstransformer.layers_t.3", "crosstransformer.layers.4", "decoder.0#0", "tdecoder.3#0"]
SAMPLES = 64


def load_package():
    name = "demucs_wgpu_amd"
    if name in sys.modules:
        return sys.modules[name]
    pkg = ROOT / "demucs-wgpu_amd"
    spec = importlib.util.spec_from_file_location(name, pkg / "__init__.py", submodule_search_locations=[str(pkg)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def key(name: str) -> str:
    return name.replace(".", "_").replace("#", "_")


def fingerprint(a: np.ndarray) -> dict:
    flat = np.asarray(a, dtype=np.float64).ravel()
    idx = np.linspace(0, flat.size - 1, SAMPLES).round().astype(np.int64)
    return {"shape": np.array(a.shape, np.int64), "sum": np.float64(flat.sum()),
            "sumsq": np.float64((flat * flat).sum()), "index": idx, "sample": flat[idx].astype(np.float32)}


def weight_checksums(weights) -> dict:
    names = sorted(weights)
    return {"weights_sum": np.array([np.float64(weights[n].astype(np.float64).sum()) for n in names]),
            "weights_names": np.array(names)}


def main():
    import torch_htdemucs as th
    dmx = load_package()

    cfg = dmx.Config()
    cfg.segment = 4096 / cfg.samplerate
    assert cfg.training_length == 4096
    weights = dmx.random_init(0, cfg)
    mix = dmx.signals.gaussian_segments(0, 1, cfg.training_length)
    trace = {}
    stems = th.forward(weights, mix, trace)
    out = {"mix": mix, "stems": stems.astype(np.float32), "segment_samples": np.int64(4096), "seed": np.int64(0)}
    out.update(weight_checksums(weights))
    for name in TRACED:
        for k, v in fingerprint(trace[name].numpy()).items():
            out[f"act_{key(name)}_{k}"] = v
    out["traced"] = np.array(TRACED)
    np.savez_compressed(HERE / "htdemucs_L4096_seed0.npz", **out)

    full = dmx.Config()
    tw = dmx.xavier_transformer_init(2, full)
    rng = np.random.default_rng(4)
    x = rng.normal(size=(1, 512, 4, 6)).astype(np.float32)
    xt = rng.normal(size=(1, 512, 12)).astype(np.float32)
    rx, rxt = th.transformer(th.Weights(tw), th.T(x), th.T(xt))
    t_out = {"x": x, "xt": xt, "out": rx.numpy().astype(np.float32), "out_t": rxt.numpy().astype(np.float32),
             "seed": np.int64(2)}
    t_out.update(weight_checksums({k: v for k, v in tw.items() if k.startswith("crosstransformer.")}))
    np.savez_compressed(HERE / "transformer_F4T6_seed2.npz", **t_out)
    for f in sorted(HERE.glob("*.npz")):
        print(f.name, f.stat().st_size, "bytes")


if __name__ == "__main__":
    main()
