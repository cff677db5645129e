"""Checkpoint readers (include/dmx_ckpt.h) against files written here by the
`safetensors` package and by `torch.save`: every tensor comes back as the f32
value of what was stored (F16/BF16 widen exactly), metadata and kwargs become
the config as `HtdemucsConfig::from_kwargs_json` reads it (config.rs:150-215),
and malformed inputs raise the reference's error kinds (safetensors.rs:38-106,
ckpt/mod.rs:57-120, ckpt/pickle.rs:140-460). Host code only: no GPU.
"""
import io
import json
import pickle
import struct
import zipfile
from collections import OrderedDict
from fractions import Fraction

import numpy as np
import pytest
import torch
from safetensors.numpy import save as st_save

from conftest import load_package

CHECKPOINT, IO, CONFIG = 9, 10, 2


@pytest.fixture(scope="module")
def ckpt():
    pkg = load_package()
    from demucs_wgpu_amd import checkpoint
    return pkg, checkpoint


def rng(seed):
    return np.random.default_rng(seed)


def ft_kwargs(segment):
    """The kwargs of an htdemucs_ft checkpoint: the default architecture plus training-only keys."""
    return {"sources": ["drums", "bass", "other", "vocals"], "audio_channels": 2, "samplerate": 44100,
            "segment": segment, "channels": 48, "growth": 2, "nfft": 4096, "depth": 4, "stride": 4,
            "kernel_size": 8, "context": 1, "freq_emb": 0.2, "emb_scale": 10, "cac": True,
            "bottom_channels": 512, "t_layers": 5, "t_heads": 8, "t_hidden_scale": 4.0, "t_max_period": 10000.0,
            "t_weight_pos_embed": 1.0, "t_weight_decay": 0.0, "t_sparse_attn_window": 400, "wiener_iters": 0}


def test_safetensors_tensors_widen_exactly_and_keep_metadata(ckpt):
    pkg, ck = ckpt
    r = rng(1)
    special = np.array([0.0, -0.0, 1.0, -2.5, 6.1e-5, 5.96e-8, -5.96e-8, 65504.0, np.inf, -np.inf, np.nan], np.float16)
    tensors = {
        "encoder.0.conv.weight": r.normal(size=(48, 4, 8, 1)).astype(np.float16),
        "decoder.3.conv_tr.bias": r.normal(size=(16,)).astype(np.float32),
        "f64": r.normal(size=(2, 3)),
        "i64": np.arange(-3, 3, dtype=np.int64),
        "i8": np.array([-128, 0, 127], np.int8),
        "u8": np.array([0, 255], np.uint8),
        "special": special,
        "scalar": np.array(3.5, np.float32),
    }
    meta = {"klass": "demucs.htdemucs.HTDemucs", "kwargs": json.dumps(ft_kwargs({"numerator": 39, "denominator": 5}))}
    loaded = ck.load_weights_from_bytes(st_save(tensors, metadata=meta), torch_zip=False)
    assert list(loaded.tensors) == sorted(tensors)
    for name, want in tensors.items():
        got = loaded.tensors[name]
        assert got.dtype == np.float32 and got.shape == want.shape, name
        np.testing.assert_array_equal(got, want.astype(np.float32), err_msg=name)
    assert loaded.metadata == meta
    assert loaded.config == pkg.Config()  # the ft kwargs are the default architecture


def test_bf16_widens_by_shifting_the_bits(ckpt):
    _, ck = ckpt
    vals = np.array([1.0, -3.140625, 1e-30, 2.0 ** 100], np.float32)
    bits = (vals.view(np.uint32) >> 16).astype("<u2")
    header = json.dumps({"x": {"dtype": "BF16", "shape": [4], "data_offsets": [0, 8]}}).encode()
    data = struct.pack("<Q", len(header)) + header + bits.tobytes()
    got = ck.load_weights_from_bytes(data, torch_zip=False).tensors["x"]
    np.testing.assert_array_equal(got, (bits.astype(np.uint32) << 16).view(np.float32))


def test_safetensors_file_by_extension_and_default_config(ckpt, tmp_path):
    pkg, ck = ckpt
    path = tmp_path / "model.safetensors"
    w = {"a": rng(2).normal(size=(3, 5)).astype(np.float32)}
    path.write_bytes(st_save(w))
    loaded = ck.load_weights(path)
    np.testing.assert_array_equal(loaded.tensors["a"], w["a"])
    assert loaded.metadata == {} and loaded.config == pkg.Config()


def torch_bytes(obj):
    buf = io.BytesIO()
    torch.save(obj, buf)
    return buf.getvalue()


def state_dict():
    g = torch.Generator().manual_seed(3)
    base = torch.randn(6, 4, generator=g)
    return OrderedDict([
        ("encoder.0.conv.weight", torch.randn(48, 4, 8, 1, generator=g).half()),
        ("encoder.0.conv.bias", torch.randn(48, generator=g)),
        ("transposed", torch.randn(5, 7, generator=g).t()),  # a strided view of its storage
        ("rows", base[1:4]),  # an offset view sharing a storage with "base"
        ("base", base),
        ("cols", base[:, 1::2]),
        ("bf16", torch.randn(9, generator=g).bfloat16()),
        ("f64", torch.randn(2, 2, generator=g).double()),
        ("steps", torch.arange(5)),
        ("param", torch.nn.Parameter(torch.randn(3, generator=g))),
    ])


def expected(t):
    return t.detach().float().numpy()


@pytest.mark.parametrize("wrap", ["bare", "state", "model_state_dict", "state_dict"])
def test_torch_zip_state_dicts_are_read_through_the_pickle(ckpt, wrap):
    pkg, ck = ckpt
    sd = state_dict()
    if wrap == "bare":
        obj = sd
    else:  # a demucs package or a training checkpoint around the state dict
        obj = {"klass": torch.nn.Linear, "args": (), "kwargs": {"segment": Fraction(39, 5), "sources": ["a"]},
               wrap: sd, "epoch": 7}
    loaded = ck.load_weights_from_bytes(torch_bytes(obj), torch_zip=True)
    assert list(loaded.tensors) == sorted(sd)
    for name, t in sd.items():
        np.testing.assert_array_equal(loaded.tensors[name], expected(t), err_msg=name)
    assert loaded.metadata == {} and loaded.config == pkg.Config()


@pytest.mark.parametrize("protocol", [0, 1, 3, 4, 5])
def test_every_pickle_protocol_torch_writes_is_read(ckpt, protocol):
    """torch.save(pickle_protocol=p): protocol 0/1 text opcodes (INT, GET,
    PUT, GLOBAL lines), protocol 4/5 frames, MEMOIZE and STACK_GLOBAL."""
    _, ck = ckpt
    sd = state_dict()
    buf = io.BytesIO()
    torch.save(sd, buf, pickle_protocol=protocol)
    loaded = ck.load_weights_from_bytes(buf.getvalue(), torch_zip=True)
    assert list(loaded.tensors) == sorted(sd)
    for name, t in sd.items():
        np.testing.assert_array_equal(loaded.tensors[name], expected(t), err_msg=name)


def test_non_tensor_entries_are_skipped_and_sparse_tensors_refused(ckpt):
    _, ck = ckpt
    sd = OrderedDict(w=torch.ones(2), none=None, obj=Fraction(1, 3))
    loaded = ck.load_weights_from_bytes(torch_bytes(sd), torch_zip=True)
    assert list(loaded.tensors) == ["w"]
    sp = torch.sparse_coo_tensor([[0, 1], [1, 0]], [1.0, 2.0], (2, 2))
    with pytest.raises(ck.CheckpointError) as e:
        ck.load_weights_from_bytes(torch_bytes(OrderedDict(w=torch.ones(2), s=sp)), torch_zip=True)
    assert e.value.code == CHECKPOINT and "only dense tensors" in str(e.value)
    with pytest.raises(ck.CheckpointError) as e:
        ck.load_weights_from_bytes(torch_bytes(OrderedDict(w=torch.ones(2), n=3)), torch_zip=True)
    assert "plain value" in str(e.value)


def test_torch_zip_file_by_extension(ckpt, tmp_path):
    _, ck = ckpt
    sd = state_dict()
    path = tmp_path / "htdemucs.th"
    torch.save(sd, path)
    loaded = ck.load_weights(path)
    for name, t in sd.items():
        np.testing.assert_array_equal(loaded.tensors[name], expected(t), err_msg=name)


def test_kwargs_override_defaults_and_ignore_unknown_keys(ckpt):
    pkg, ck = ckpt
    assert ck.config_from_kwargs(json.dumps(ft_kwargs(7.8))) == pkg.Config()
    cfg = ck.config_from_kwargs(json.dumps({"channels": 32, "depth": 3, "t_layers": 3, "cac": False,
                                            "segment": {"numerator": 10, "denominator": 1}, "sources": ["x", "y"],
                                            "freq_emb": 0, "whatever": {"nested": [1, 2, None]}}))
    want = pkg.Config(channels=32, depth=3, t_layers=3, cac=0, segment=10.0, sources=2, freq_emb=0.0)
    assert cfg == want
    assert ck.config_from_kwargs("{}") == pkg.Config()


@pytest.mark.parametrize("text", ['{"channels": -1}', '{"channels": 1.5}', '{"cac": 1}', '{"sources": "ab"}',
                                  '{"segment": "7.8"}', '[1, 2]', 'not json', '{"channels": 48,}'])
def test_bad_kwargs_are_config_errors(ckpt, text):
    _, ck = ckpt
    with pytest.raises(ck.CheckpointError) as e:
        ck.config_from_kwargs(text)
    assert e.value.code == CONFIG


def st_raw(header, data=b""):
    h = json.dumps(header).encode()
    return struct.pack("<Q", len(h)) + h + data


@pytest.mark.parametrize("data,message", [
    (b"\x01\x02\x03", "cannot hold the 8-byte header size"),
    (struct.pack("<Q", 1000) + b"{}", "announces 1000 bytes"),
    (struct.pack("<Q", 5) + b"{oops", "JSON"),
    (st_raw({"x": {"dtype": "F32", "shape": [3], "data_offsets": [0, 8]}}, b"\0" * 8), "takes 12 bytes, but its entry spans 8"),
    (st_raw({"x": {"dtype": "F32", "shape": [1], "data_offsets": [4, 8]}}, b"\0" * 4), "lie beyond the 4-byte data section"),
    (st_raw({"x": {"dtype": "F8_E4M3", "shape": [1], "data_offsets": [0, 1]}}, b"\0"), "element type `F8_E4M3`"),
    (st_raw({"x": {"shape": [1], "data_offsets": [0, 4]}}, b"\0" * 4), "lacks a `dtype` string"),
    (st_raw({"x": {"dtype": "F32", "shape": [1], "data_offsets": [0]}}, b"\0" * 4), "must be the pair [begin, end]"),
])
def test_malformed_safetensors_are_checkpoint_errors(ckpt, data, message):
    _, ck = ckpt
    with pytest.raises(ck.CheckpointError) as e:
        ck.load_weights_from_bytes(data, torch_zip=False)
    assert e.value.code == CHECKPOINT and message in str(e.value)


def zip_bytes(entries, method=zipfile.ZIP_STORED):
    buf = io.BytesIO()
    with zipfile.ZipFile(buf, "w", method) as z:
        for name, data in entries.items():
            z.writestr(name, data)
    return buf.getvalue()


@pytest.mark.parametrize("data,message", [
    (b"not a zip at all, but long enough to scan", "not a zip archive"),
    (zip_bytes({"archive/other": b"x"}), "no `<root>/data.pkl` entry"),
    (zip_bytes({"archive/data.pkl": pickle.dumps({"a": 1}, protocol=2)}), "holds a tensor"),
    (zip_bytes({"archive/data.pkl": b"\x80\x02\xff."}), "opcode 0xff is not one this reader runs"),
    (zip_bytes({"archive/data.pkl": b"\x80\x02}q\x00(X\x01\x00\x00\x00a"}), "ends before a STOP opcode"),
    (zip_bytes({"archive/data.pkl": pickle.dumps({"a": 1}, protocol=2)}, zipfile.ZIP_DEFLATED), "compressed"),
])
def test_malformed_torch_zips_are_checkpoint_errors(ckpt, data, message):
    _, ck = ckpt
    with pytest.raises(ck.CheckpointError) as e:
        ck.load_weights_from_bytes(data, torch_zip=True)
    assert e.value.code == CHECKPOINT and message in str(e.value)


def test_a_missing_storage_blob_is_reported(ckpt):
    _, ck = ckpt
    src = zipfile.ZipFile(io.BytesIO(torch_bytes(OrderedDict(w=torch.ones(3)))))
    kept = {n: src.read(n) for n in src.namelist() if "/data/" not in n}
    with pytest.raises(ck.CheckpointError) as e:
        ck.load_weights_from_bytes(zip_bytes(kept), torch_zip=True)
    assert "lacks the storage entry" in str(e.value)


def test_a_missing_file_is_an_io_error(ckpt, tmp_path):
    _, ck = ckpt
    with pytest.raises(ck.CheckpointError) as e:
        ck.load_weights(tmp_path / "absent.safetensors")
    assert e.value.code == IO
