"""dmx_op_spec_normalise_noalloc: the STFT front end with its frames and
moments in the library's fixed device scratch instead of allocated memory.
Checked through the C-ABI against dmx_op_spec_normalise on two calls in a
row, the second smaller (the scratch keeps the first call's contents), and
for its size limit."""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _run(lib, name, mix, stream):
    b, _, L = mix.shape
    le = -(-L // 1024)
    xspec = torch.empty((b, 4, 2048, le), device="cuda")
    xwave = torch.empty((b, 2, L), device="cuda")
    norms = torch.empty((b, 4), device="cuda")
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    rc = getattr(lib, name)(ctypes.c_void_p(stream), P(mix), b, L, P(xspec), P(xwave), P(norms))
    assert rc == 0, lib.dmx_last_error()
    return xspec, xwave, norms


def _rms_rel(ref, got):
    ref = ref.double()
    return float(torch.sqrt(torch.mean((ref - got.double()) ** 2)) / torch.sqrt(torch.mean(ref ** 2)))


def test_noalloc_front_end_matches_the_allocating_one(dmx):
    lib = dmx._native.load()
    stream = torch.cuda.current_stream().cuda_stream
    g = torch.Generator(device="cuda").manual_seed(5)
    for b, L in ((2, 343980), (1, 100000)):  # the largest input the scratch takes, then a smaller one
        mix = 0.1 * torch.randn((b, 2, L), device="cuda", generator=g)
        torch.cuda.synchronize()
        ref = _run(lib, "dmx_op_spec_normalise", mix, stream)
        got = _run(lib, "dmx_op_spec_normalise_noalloc", mix, stream)
        torch.cuda.synchronize()
        for r, o in zip(ref, got):
            assert torch.isfinite(o).all()
            assert _rms_rel(r, o) <= 1e-6, (b, L, _rms_rel(r, o))
        torch.testing.assert_close(got[2], ref[2], rtol=1e-6, atol=0.0)


def test_noalloc_front_end_refuses_inputs_beyond_its_scratch(dmx):
    lib = dmx._native.load()
    mix = torch.zeros((3, 2, 343980), device="cuda")  # 3 x 336 frames > 672
    out = torch.empty(1, device="cuda")
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    rc = lib.dmx_op_spec_normalise_noalloc(None, P(mix), 3, 343980, P(out), P(out), P(out))
    assert rc == 1  # DMX_ERR_SHAPE, before any launch
    assert b"fixed scratch" in lib.dmx_last_error()
