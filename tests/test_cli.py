"""The command line's host-only commands on the CPU: `info`, `compare`, the
device words and the bench input (crates/demucs-cli/src/main.rs:66-88,
:224-301, :1130-1135)."""
import numpy as np
import pytest

from conftest import load_package

dmx = load_package()
from demucs_wgpu_amd import cli  # noqa: E402  (registered by load_package)


def test_info_prints_the_parameter_count_and_layer_table(capsys):
    assert cli.main(["info", "--model", "random:0"]) == 0
    out = capsys.readouterr().out
    assert "41984456 parameters" in out
    assert "encoder.0  2048 bins,   4 ->  48 channels, k=8 s=4 p=2" in out
    assert "bottleneck: 8 bins, 384 channels" in out
    assert "decoder.3  48 ->  16 channels" in out


def test_compare_reports_the_fixtures_snr(tmp_path, capsys):
    x = np.random.default_rng(0).normal(size=(2, 1000)).astype(np.float32)
    dmx.audio.write_wav_f32(tmp_path / "a.wav", 44100, x)
    dmx.audio.write_wav_f32(tmp_path / "b.wav", 44100, x + np.float32(1e-3))
    assert cli.main(["compare", str(tmp_path / "a.wav"), str(tmp_path / "b.wav")]) == 0
    out = capsys.readouterr().out
    rms = float(np.sqrt(np.mean(x.astype(np.float64) ** 2)))
    assert f"{-20 * np.log10(1e-3 / rms):.2f} dB SNR" in out


def test_compare_refuses_different_shapes(tmp_path, capsys):
    dmx.audio.write_wav_f32(tmp_path / "a.wav", 44100, np.zeros((2, 10), np.float32))
    dmx.audio.write_wav_f32(tmp_path / "b.wav", 44100, np.zeros((2, 11), np.float32))
    assert cli.main(["compare", str(tmp_path / "a.wav"), str(tmp_path / "b.wav")]) == 1
    assert "shape mismatch: 2x10 vs 2x11" in capsys.readouterr().err


@pytest.mark.parametrize("spec, kind, device", [("auto", "auto", 0), ("gpu", "hip", 0), ("HIP:3", "hip", 3)])
def test_device_words(spec, kind, device):
    b = cli.parse_device(spec)
    assert (b.kind, b.device) == (kind, device)


def test_cpu_device_is_refused():
    with pytest.raises(cli.CliError):
        cli.parse_device("cpu")


def test_unknown_stem_fails_before_loading(tmp_path, capsys):
    assert cli.main(["separate", str(tmp_path / "x.wav"), "-o", str(tmp_path), "--stem", "guitar"]) == 1
    assert "must be one of" in capsys.readouterr().err


def test_bench_input_is_the_reference_lcg():
    x = cli.bench_mix(2, 3)
    state, want = 12345, []
    for _ in range(6):
        state = (state * 1664525 + 1013904223) % (1 << 32)
        want.append(np.float32(((state >> 8) / 8388608.0 - 1.0) * 0.1))
    assert x.reshape(-1).tolist() == want
