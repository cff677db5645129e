"""The command line (crates/demucs-cli/src/main.rs) on the device: `separate`
writes float WAV stems equal to the library's separation, with --stem and
--two-stems companions, and `bench` times a segment."""
import numpy as np
import pytest

from conftest import load_package, snr_db

load_package()
from demucs_wgpu_amd import cli  # noqa: E402  (registered by load_package)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def track(dmx, tmp_path_factory):
    d = tmp_path_factory.mktemp("cli")
    mix = dmx.signals.synthetic_mix(11, 9.0)
    path = d / "mix.wav"
    dmx.audio.write_wav_f32(path, 44100, mix)
    return d, path, dmx.audio.read_audio(path).data


def reference(dmx, mix, shifts=0, wanted=None):
    cfg = dmx.Config()
    runner = dmx.Runner(dmx.random_init(3, cfg), cfg)
    opts = dmx.SeparateOptions(shifts=shifts, overlap=0.25, batch_chunks=8)
    return dmx.separate_runners([runner], mix[0], mix[1], 44100, opts, wanted=wanted)


def test_separate_writes_every_stem(dmx, track, capsys):
    d, path, mix = track
    out = d / "all"
    assert cli.main(["separate", str(path), "-o", str(out), "--model", "random:3", "--shifts", "0"]) == 0
    text = capsys.readouterr().out
    assert "RTFx" in text and "wrote" in text
    ref = reference(dmx, mix)
    for s, name in enumerate(dmx.Config.SOURCES):
        a = dmx.audio.read_audio(out / f"{name}.wav")
        assert a.sample_rate == 44100 and a.data.shape == (2, mix.shape[1])
        assert snr_db(ref[s], a.data) > 120.0, name


def test_two_stems_companions(dmx, track):
    d, path, mix = track
    ref = reference(dmx, mix)
    out = d / "two"
    assert cli.main(["separate", str(path), "-o", str(out), "--model", "random:3", "--shifts", "0",
                         "--two-stems", "vocals"]) == 0
    vocals = dmx.audio.read_audio(out / "vocals.wav").data
    rest = dmx.audio.read_audio(out / "no_vocals.wav").data
    assert snr_db(ref[3], vocals) > 120.0
    assert snr_db(ref[0] + ref[1] + ref[2], rest) > 100.0
    out = d / "minus"
    assert cli.main(["separate", str(path), "-o", str(out), "--model", "random:3", "--shifts", "0",
                         "--two-stems", "vocals", "--other-method", "minus"]) == 0
    minus = dmx.audio.read_audio(out / "minus_vocals.wav").data
    assert snr_db(mix - ref[3], minus) > 100.0


def test_single_stem_to_one_file(dmx, track):
    d, path, mix = track
    out = d / "drums_only.wav"
    assert cli.main(["separate", str(path), "-o", str(out), "--model", "random:3", "--shifts", "0",
                         "--stem", "drums"]) == 0
    ref = reference(dmx, mix, wanted=[True, False, False, False])
    assert snr_db(ref[0], dmx.audio.read_audio(out).data) > 120.0


def test_separate_rejects_a_wrong_rate(dmx, track, capsys):
    d, _, mix = track
    p = d / "m22.wav"
    dmx.audio.write_wav_f32(p, 22050, mix[:, :22050])
    assert cli.main(["separate", str(p), "-o", str(d / "x"), "--model", "random:3"]) == 1
    assert "22050 Hz but the model wants 44100 Hz" in capsys.readouterr().err


def test_bench_times_a_segment(dmx, capsys):
    assert cli.main(["bench", "--model", "random:0", "--repeats", "2"]) == 0
    text = capsys.readouterr().out
    assert "chunk forward" in text and "x raw" in text
