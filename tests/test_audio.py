"""WAV files and the comparison metric (include/dmx_audio.h), on the CPU.

The cases restate the reference's own tests (crates/demucs-core/src/audio.rs:
737-958, crates/demucs-core/src/fixtures.rs:198-233) on byte strings built
here, and pin the codec independently with scipy.io.wavfile, which writes and
reads the same files by its own implementation.
"""
import struct

import numpy as np
import pytest
import scipy.io.wavfile as wavfile

from conftest import load_package

dmx = load_package()
audio = dmx.audio


def riff(fmt_tag, channels, rate, bits, payload, extra_chunks=b"", extensible_tag=None):
    """A WAV byte string: RIFF header, optional chunks, fmt, data."""
    align = channels * bits // 8
    if extensible_tag is None:
        fmt = struct.pack("<HHIIHH", fmt_tag, channels, rate, rate * align, align, bits)
    else:
        guid_tail = bytes.fromhex("000000001000800000aa00389b71")
        fmt = struct.pack("<HHIIHHHHI", 0xFFFE, channels, rate, rate * align, align, bits, 22, bits, 0) + \
            struct.pack("<H", extensible_tag) + guid_tail
    body = b"WAVE" + extra_chunks + b"fmt " + struct.pack("<I", len(fmt)) + fmt + \
        b"data" + struct.pack("<I", len(payload)) + payload
    return b"RIFF" + struct.pack("<I", len(body)) + body


def write_bytes(tmp_path, name, data):
    p = tmp_path / name
    p.write_bytes(data)
    return p


def test_reads_mono_float_wav_channel_major(tmp_path):
    p = write_bytes(tmp_path, "m.wav", riff(3, 1, 44100, 32, np.array([0.5, -0.25, 0.125], "<f4").tobytes()))
    a = audio.read_audio(p)
    assert (a.channels, a.samples, a.sample_rate) == (1, 3, 44100)
    assert a.channel(0).tolist() == [0.5, -0.25, 0.125]


def test_deinterleaves_stereo(tmp_path):
    p = write_bytes(tmp_path, "s.wav", riff(3, 2, 44100, 32, np.array([1, 2, 3, 4], "<f4").tobytes()))
    a = audio.read_audio(p)
    assert a.channel(0).tolist() == [1.0, 3.0] and a.channel(1).tolist() == [2.0, 4.0]


def test_reads_pcm16_scaled_like_soundfile(tmp_path):
    p = write_bytes(tmp_path, "p16.wav", riff(1, 1, 44100, 16, np.array([32767, -32768, 0], "<i2").tobytes()))
    x = audio.read_audio(p).channel(0)
    assert abs(x[0] - 0.9999695) < 1e-6 and x[1] == -1.0 and x[2] == 0.0


def test_reads_pcm24_with_sign_extension(tmp_path):
    p = write_bytes(tmp_path, "p24.wav", riff(1, 1, 44100, 24, bytes([0x00, 0x00, 0x80, 0xFF, 0xFF, 0x7F])))
    x = audio.read_audio(p).channel(0)
    assert x[0] == -1.0 and abs(x[1] - 0.99999988) < 1e-6


def test_reads_pcm32_and_float64(tmp_path):
    p = write_bytes(tmp_path, "p32.wav", riff(1, 1, 8000, 32, np.array([1 << 30, -(1 << 31)], "<i4").tobytes()))
    assert audio.read_audio(p).channel(0).tolist() == [0.5, -1.0]
    p = write_bytes(tmp_path, "f64.wav", riff(3, 1, 8000, 64, np.array([0.1, -3.0], "<f8").tobytes()))
    assert audio.read_audio(p).channel(0).tolist() == [np.float32(0.1), -3.0]


def test_extensible_format_is_resolved_by_its_subformat(tmp_path):
    pcm = riff(None, 2, 48000, 24, bytes([0, 0, 0x40, 0, 0, 0xC0]), extensible_tag=1)
    a = audio.read_audio(write_bytes(tmp_path, "ext_pcm.wav", pcm))
    assert a.channel(0).tolist() == [0.5] and a.channel(1).tolist() == [-0.5] and a.sample_rate == 48000
    flt = riff(None, 1, 48000, 32, np.array([0.25], "<f4").tobytes(), extensible_tag=3)
    assert audio.read_audio(write_bytes(tmp_path, "ext_f.wav", flt)).channel(0).tolist() == [0.25]


def test_chunks_between_fmt_and_data_are_skipped(tmp_path):
    extra = b"LIST" + struct.pack("<I", 5) + b"abcde" + b"\x00" + b"fact" + struct.pack("<I", 4) + b"\x03\x00\x00\x00"
    p = write_bytes(tmp_path, "c.wav", riff(3, 1, 44100, 32, np.array([0.5, 1.5, -2], "<f4").tobytes(), extra))
    assert audio.read_audio(p).channel(0).tolist() == [0.5, 1.5, -2.0]


@pytest.mark.parametrize("data, why", [
    (b"not a wav file at all", "not a RIFF/WAVE"),
    (riff(1, 1, 44100, 8, bytes([1, 2, 3])), "unsupported WAV encoding"),
    (riff(2, 1, 44100, 16, b"\0\0"), "unsupported WAV encoding"),
    (riff(1, 2, 44100, 16, b"\0\0\0"), "not a whole number"),
    (b"RIFF" + struct.pack("<I", 4) + b"WAVE", "missing fmt chunk"),
])
def test_rejects_what_it_cannot_read(tmp_path, data, why):
    p = write_bytes(tmp_path, "bad.wav", data)
    with pytest.raises(dmx.DmxError) as e:
        audio.read_audio(p)
    assert e.value.kind == "Audio" and why in str(e.value)


def test_missing_file_is_an_io_error(tmp_path):
    with pytest.raises(dmx.DmxError) as e:
        audio.probe_audio(tmp_path / "absent.wav")
    assert e.value.kind == "Io"


def test_mono_is_duplicated_for_stereo_configs():
    a = audio.Audio(44100, np.array([[0.5, -0.5]], np.float32)).ensure_channels(2)
    assert a.channels == 2 and a.channel(1).tolist() == [0.5, -0.5]
    with pytest.raises(dmx.DmxError):
        audio.Audio(44100, np.zeros((3, 2), np.float32)).ensure_channels(2)


def test_round_trips_through_the_writer(tmp_path):
    p = tmp_path / "rt.wav"
    audio.write_wav_f32(p, 22050, np.array([[0.25, -0.75], [1.0, -1.0]], np.float32))
    a = audio.read_audio(p)
    assert a.sample_rate == 22050 and a.data.tolist() == [[0.25, -0.75], [1.0, -1.0]]


def test_writer_interleaves_frames_on_disk(tmp_path):
    p = tmp_path / "il.wav"
    audio.write_wav_f32(p, 8000, np.array([[1, 2], [3, 4]], np.float32))
    raw = p.read_bytes()
    at = raw.index(b"data") + 8
    assert np.frombuffer(raw[at:at + 16], "<f4").tolist() == [1.0, 3.0, 2.0, 4.0]


def test_probe_audio_matches_decoded_frames(tmp_path):
    p = tmp_path / "probe.wav"
    audio.write_wav_f32(p, 8000, np.array([[1, 2], [3, 4]], np.float32))
    info, a = audio.probe_audio(p), audio.read_audio(p)
    assert (info.sample_rate, info.channels, info.frames) == (a.sample_rate, a.channels, a.samples)


def test_float_wav_writer_matches_write_wav_f32(tmp_path):
    cm = np.array([[0.25, -0.75, 0.5], [1.0, -1.0, 0.0]], np.float32)
    audio.write_wav_f32(tmp_path / "bulk.wav", 22050, cm)
    with audio.FloatWavWriter(tmp_path / "stream.wav", 22050, 2) as w:
        w.write_frame([0.25, 1.0])
        w.write_interleaved(np.array([-0.75, -1.0], np.float32))
        w.write_planar(cm[:, 2:])
        assert w.frames_written() == 3
    assert (tmp_path / "bulk.wav").read_bytes() == (tmp_path / "stream.wav").read_bytes()


def test_pcm_quantisation_rounds_half_away_and_clips(tmp_path):
    x = np.array([[0.0, 0.5, -0.5, 1.0, -1.0, 2.0, -2.0, 1.5 / 32768, -1.5 / 32768, np.nan]], np.float32)
    audio.write_wav(tmp_path / "q.wav", audio.Subtype.PCM_16, 8000, x)
    rate, got = wavfile.read(tmp_path / "q.wav")
    assert rate == 8000 and got.dtype == np.int16
    assert got.tolist() == [0, 16384, -16384, 32767, -32768, 32767, -32768, 2, -2, 0]


def test_written_files_read_back_by_scipy(tmp_path):
    r = np.random.default_rng(3)
    x = (r.uniform(-1.2, 1.2, size=(2, 500))).astype(np.float32)
    audio.write_wav(tmp_path / "f.wav", audio.Subtype.FLOAT, 44100, x)
    rate, got = wavfile.read(tmp_path / "f.wav")
    assert rate == 44100 and np.array_equal(got.T, x)
    audio.write_wav(tmp_path / "i16.wav", audio.Subtype.PCM_16, 44100, x)
    _, got16 = wavfile.read(tmp_path / "i16.wav")
    expect16 = np.clip(np.where(x * 32768 >= 0, np.floor(x * 32768 + 0.5), np.ceil(x * 32768 - 0.5)), -32768, 32767)
    assert np.array_equal(got16.T.astype(np.float64), expect16)
    audio.write_wav(tmp_path / "i24.wav", audio.Subtype.PCM_24, 44100, x)
    _, got24 = wavfile.read(tmp_path / "i24.wav")
    scale = 1 << 23
    expect24 = np.clip(np.where(x * scale >= 0, np.floor(x * scale + 0.5), np.ceil(x * scale - 0.5)), -scale, scale - 1)
    # scipy returns 24-bit PCM left-justified in int32
    assert np.array_equal((got24.T.astype(np.int64) >> 8).astype(np.float64), expect24)


@pytest.mark.parametrize("dtype, scale", [(np.int16, 32768.0), (np.int32, 2147483648.0), (np.float32, 1.0),
                                          (np.float64, 1.0)])
def test_reads_files_scipy_wrote(tmp_path, dtype, scale):
    r = np.random.default_rng(4)
    if np.issubdtype(dtype, np.integer):
        info = np.iinfo(dtype)
        data = r.integers(info.min, info.max, size=(300, 2), endpoint=True).astype(dtype)
    else:
        data = r.normal(size=(300, 2)).astype(dtype)
    wavfile.write(tmp_path / "s.wav", 16000, data)
    a = audio.read_audio(tmp_path / "s.wav")
    assert a.sample_rate == 16000 and a.data.shape == (2, 300)
    assert np.array_equal(a.data, (data.T.astype(np.float64) / scale).astype(np.float32))


def test_comparison_reports_scale_relative_error():
    r = audio.compare([1.0, 2.0, 3.0], [1.0, 2.0, 3.0003])
    assert r.elements == 3 and abs(r.max_abs - 0.0003) < 1e-7 and r.max_abs_index == 2
    assert r.normalized_error() < 1e-4


def test_comparison_rejects_length_mismatches():
    with pytest.raises(dmx.DmxError):
        audio.compare([1.0, 2.0], [1.0])


def test_identical_buffers_have_zero_error():
    r = audio.compare([0.5, -0.25], [0.5, -0.25])
    assert r.max_abs == 0.0 and r.max_rel == 0.0 and r.snr_db() == float("inf")


def test_snr_is_the_mean_abs_error_over_the_reference_rms():
    # a constant offset c: mean |err| = c exactly, so snr = -20 log10(c / rms)
    x = np.random.default_rng(5).normal(size=4096).astype(np.float32)
    c = np.float32(0.01)
    r = audio.compare(x, x + c)
    rms = float(np.sqrt(np.mean(x.astype(np.float64) ** 2)))
    assert abs(r.mean_abs - c) < 1e-6 and abs(r.reference_rms - rms) < 1e-6
    assert abs(r.snr_db() - (-20.0 * np.log10(float(c) / rms))) < 1e-3
    assert abs(r.rms_relative_error() - float(c) / rms) < 1e-6
