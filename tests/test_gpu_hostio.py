"""The host-memory entry points: `dmx_separate` (host mix in, host stems out,
read back region by region while later chunk groups compute) against the
device-resident `dmx_separate_device`, progress reporting, and the
SegmentForward staging slots of `dmx_forward_start` / `dmx_forward_collect`
(crates/demucs-core/src/demucs/pipeline.rs:178-190, :584-619).
"""
import ctypes

import numpy as np
import pytest
import torch

from conftest import small_config, snr_db

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def small(dmx):
    cfg = small_config(dmx, 11025)
    weights = dmx.random_init(0, cfg)
    return cfg, dmx.Runner(weights, cfg)


def separate_host(dmx, runners, mix, opts, stems_out, wanted=None, progress=None):
    lib = dmx._native.load()
    handles = (ctypes.c_void_p * len(runners))(*[r.handle for r in runners])
    mask = None if wanted is None else (ctypes.c_uint8 * 4)(*[1 if w else 0 for w in wanted])
    left, right = np.ascontiguousarray(mix[0]), np.ascontiguousarray(mix[1])
    cb = dmx._native.PROGRESS(progress) if progress else dmx._native.PROGRESS()
    c_opts = opts.to_c()
    rc = lib.dmx_separate(handles, None, len(runners), mask, left.ctypes.data_as(ctypes.c_void_p),
                          right.ctypes.data_as(ctypes.c_void_p), left.shape[0], 44100, ctypes.byref(c_opts), cb,
                          None, stems_out.ctypes.data_as(ctypes.c_void_p))
    assert rc == 0, dmx._native.last_error()


def separate_device(dmx, runners, mix, opts):
    lib = dmx._native.load()
    handles = (ctypes.c_void_p * len(runners))(*[r.handle for r in runners])
    d_mix = torch.from_numpy(np.ascontiguousarray(mix)).cuda()
    d_out = torch.zeros((4, 2, mix.shape[1]), device="cuda")
    torch.cuda.synchronize()
    c_opts = opts.to_c()
    rc = lib.dmx_separate_device(handles, None, len(runners), None, ctypes.c_void_p(d_mix.data_ptr()), mix.shape[1],
                                 44100, ctypes.byref(c_opts), dmx._native.PROGRESS(), None,
                                 ctypes.c_void_p(d_out.data_ptr()))
    assert rc == 0, dmx._native.last_error()
    runners[0].synchronize()
    return d_out.cpu().numpy()


@pytest.mark.parametrize("seconds,shifts,group", [(1.3, 0, 2), (2.05, 1, 3), (1.7, 2, 2), (0.2, 0, 1)])
def test_host_separation_equals_the_device_separation(dmx, small, seconds, shifts, group):
    """The same chunk loop with the stems read back region by region (each
    group's finished samples while later groups compute) and with the stems
    left in HBM: identical up to the f64 atomics' summation order of the mix
    moments. Mix lengths leave short last regions; shifts 2 runs the
    accumulate-then-finish pass modes."""
    cfg, runner = small
    mix = dmx.signals.synthetic_mix(21, seconds)
    opts = dmx.SeparateOptions(shifts=shifts, overlap=0.25, batch_chunks=group)
    host = np.full((4, 2, mix.shape[1]), np.nan, np.float32)
    separate_host(dmx, [runner], mix, opts, host)
    dev = separate_device(dmx, [runner], mix, opts)
    assert np.isfinite(host).all()
    for s in range(4):
        assert snr_db(dev[s], host[s]) >= 120.0, (s, snr_db(dev[s], host[s]))


def test_calls_beyond_the_pinned_limit_go_through_the_ring(dmx, small, monkeypatch):
    """With DMX_PINNED_MAX_MB=0 nothing fits the pinned staging: the mix goes
    up and the stems come back through the 24 MB ring, after the last group."""
    cfg, runner = small
    mix = dmx.signals.synthetic_mix(24, 1.3)
    opts = dmx.SeparateOptions(shifts=1, overlap=0.25, batch_chunks=2)
    staged = np.zeros((4, 2, mix.shape[1]), np.float32)
    separate_host(dmx, [runner], mix, opts, staged, wanted=[True, False, True, True])
    monkeypatch.setenv("DMX_PINNED_MAX_MB", "0")
    ring = np.zeros_like(staged)
    separate_host(dmx, [runner], mix, opts, ring, wanted=[True, False, True, True])
    assert not ring[1].any()
    for s in (0, 2, 3):
        assert snr_db(staged[s], ring[s]) >= 120.0


def test_unwanted_rows_are_left_untouched(dmx, small):
    cfg, runner = small
    mix = dmx.signals.synthetic_mix(22, 1.0)
    opts = dmx.SeparateOptions(shifts=0, batch_chunks=2)
    out = np.full((4, 2, mix.shape[1]), 7.0, np.float32)
    separate_host(dmx, [runner], mix, opts, out, wanted=[False, True, False, False])
    assert (out[0] == 7.0).all() and (out[2:] == 7.0).all()
    full = np.zeros_like(out)
    separate_host(dmx, [runner], mix, opts, full)
    assert snr_db(full[1], out[1]) >= 120.0


def test_progress_counts_every_chunk_and_keeps_the_schedule(dmx, small):
    """Progress comes from host waits on per-group marks: it reaches the
    total, never goes back, and the stems match a run without a callback."""
    cfg, runner = small
    mix = dmx.signals.synthetic_mix(23, 1.6)
    opts = dmx.SeparateOptions(shifts=1, overlap=0.25, batch_chunks=2)
    seen = []
    a = np.zeros((4, 2, mix.shape[1]), np.float32)
    separate_host(dmx, [runner], mix, opts, a, progress=lambda d, t, u: seen.append((d, t)))
    b = np.zeros_like(a)
    separate_host(dmx, [runner], mix, opts, b)
    stride = int(0.75 * cfg.training_length)
    assert seen and seen[-1][0] == seen[-1][1]
    assert all(x[0] < y[0] for x, y in zip(seen, seen[1:]))
    assert seen[-1][1] >= -(-mix.shape[1] // stride)
    for s in range(4):
        assert snr_db(a[s], b[s]) >= 120.0


def test_forward_groups_in_flight_reuse_staging(dmx, small):
    """Three groups queued before any is collected (the third of a larger
    batch, which grows a staging slot), collected out of order, then the
    same again: each result equals the synchronous forward of its input."""
    cfg, runner = small
    L = cfg.training_length
    inputs = [dmx.signals.gaussian_segments(30 + i, b, L) for i, b in enumerate((1, 2, 3))]
    ref = [runner.forward(x) for x in inputs]
    for _ in range(2):
        pending = [runner.start(x) for x in inputs]
        outs = {}
        for i in (1, 0, 2):
            outs[i] = runner.collect(pending[i])
        for i in range(3):
            np.testing.assert_array_equal(outs[i], ref[i])


def test_collect_rejects_another_runners_group(dmx, small):
    cfg, runner = small
    other = dmx.Runner(dmx.random_init(1, cfg), cfg)
    p = runner.start(dmx.signals.gaussian_segments(40, 1, cfg.training_length))
    with pytest.raises(dmx.DmxError) as e:
        other.collect(p)
    assert e.value.kind == "Argument"
    runner.collect(p)


@pytest.mark.parametrize("seconds,shifts,group,pinned_mb", [(2.05, 1, 3, None), (1.7, 2, 2, None),
                                                            (1.3, 0, 2, "0")])
def test_emit_hands_over_the_separation_region_by_region(dmx, small, monkeypatch, seconds, shifts, group,
                                                         pinned_mb):
    """dmx_separate_emit (separate_emit / separate_streaming_normalized_mix,
    crates/demucs-core/src/api.rs:265-298, :697-785): the regions come in
    order, tile [0, samples) exactly, and hold dmx_separate's stems; rows of
    unwanted stems are null. pinned_mb = 0 takes the path for mixes longer
    than the pinned staging (regions after the chunk loop)."""
    if pinned_mb is not None:
        monkeypatch.setenv("DMX_PINNED_MAX_MB", pinned_mb)
    cfg, runner = small
    mix = dmx.signals.synthetic_mix(5, seconds)
    opts = dmx.SeparateOptions(shifts=shifts, overlap=0.25, batch_chunks=group)
    wanted = [True, False, True, True]
    ref = np.zeros((4, 2, mix.shape[1]), np.float32)
    separate_host(dmx, [runner], mix, opts, ref, wanted=wanted)
    got = np.full((4, 2, mix.shape[1]), np.nan, np.float32)
    regions = []
    progress = []

    def on_frames(start, block):
        regions.append((start, block.shape[-1]))
        got[:, :, start:start + block.shape[-1]] = block

    dmx.separate_emit_runners([runner], mix[0], mix[1], 44100, opts, on_frames, wanted=wanted,
                              on_progress=lambda p: progress.append((p.done, p.total)))
    assert regions[0][0] == 0 and sum(n for _, n in regions) == mix.shape[1]
    assert all(a + n == b for (a, n), (b, _) in zip(regions, regions[1:]))
    if pinned_mb is None:
        assert len(regions) >= 2  # regions flushed while later groups computed
    assert not got[1].any()  # the unwanted stem's rows come as zeros
    for s in (0, 2, 3):
        assert snr_db(ref[s], got[s]) > 120.0, s
    assert progress and progress[-1][0] == progress[-1][1]


def test_emit_callback_error_stops_the_separation(dmx, small):
    cfg, runner = small
    mix = dmx.signals.synthetic_mix(6, 2.05)
    opts = dmx.SeparateOptions(shifts=0, overlap=0.25, batch_chunks=2)
    calls = []

    def on_frames(start, block):
        calls.append(start)
        raise KeyError("disk full")

    with pytest.raises(KeyError):
        dmx.separate_emit_runners([runner], mix[0], mix[1], 44100, opts, on_frames)
    assert len(calls) == 1
    # the runner is usable afterwards
    out = dmx.separate_runners([runner], mix[0], mix[1], 44100, opts)
    assert np.isfinite(out).all()
