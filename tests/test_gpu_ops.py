"""Per-kernel parity: each HIP kernel through include/dmx_ops.h against the CPU
oracle on the same seeded inputs, at the reference's own gates
(core/tests/gpu_*.rs): rms-relative <= 1e-5 for contractions, <= 1e-6 for
norms/elementwise (relaxed where noted for the f32 FFT), exact for data movement.
"""
import ctypes

import numpy as np
import pytest

from conftest import rms_relative_error, snr_db

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def rng(seed):
    return np.random.default_rng(seed)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).cuda()


def ptr(t):
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


@pytest.fixture(params=[0, 2], ids=["fp32_planes", "fp32_mfma"])
def fp32_precision(lib, request):
    """Both fp32 settings of dmx_op_set_precision: the default (linears,
    attention and the wide-tile convolutions on three bf16 planes per
    operand) and fp32 MFMA everywhere."""
    assert lib.dmx_op_set_precision(request.param) == 0
    yield request.param
    assert lib.dmx_op_set_precision(0) == 0


@pytest.fixture(scope="module")
def lib(dmx):
    from demucs_wgpu_amd import _native
    return _native.load()


def call(lib, name, *args):
    rc = getattr(lib, name)(*args)
    torch.cuda.synchronize()
    if rc != 0:
        raise RuntimeError(f"{name}: {lib.dmx_last_error().decode()}")


@pytest.mark.parametrize("rows,k,n,tail", [(300, 512, 1536, 0), (37, 19, 70, 0), (64, 512, 2048, 1),
                                           (129, 2048, 512, 2), (2688, 512, 512, 2)])
def test_linear_matches_oracle(lib, oracle, fp32_precision, rows, k, n, tail):
    r = rng(rows + k + n)
    x = r.uniform(-0.4, 0.4, (rows, k)).astype(np.float32)
    w = r.uniform(-0.4, 0.4, (n, k)).astype(np.float32)
    b = r.uniform(-0.4, 0.4, n).astype(np.float32)
    res = r.uniform(-1, 1, (rows, n)).astype(np.float32)
    g = r.uniform(0.1, 0.5, n).astype(np.float32)
    ref = oracle.sgemm(x, w.T) + b
    if tail == 1:
        ref = oracle.gelu(ref)
    elif tail == 2:
        ref = res + ref * g
    dx, dw, db, dres, dg = dev(x), dev(w), dev(b), dev(res), dev(g)
    out = torch.empty((rows, n), device="cuda")
    call(lib, "dmx_op_linear", stream(), ptr(dx), rows, k, ptr(dw), ptr(db), n, tail, ptr(dres), ptr(dg), ptr(out))
    assert rms_relative_error(ref, out.cpu().numpy()) < 1e-5


@pytest.mark.parametrize("b,ic,h,w,oc,kh,kw,sh,sw,ph,pw,dh,dw", [
    (1, 4, 64, 9, 48, 8, 1, 4, 1, 2, 0, 1, 1),      # freq encoder conv (k(8,1) s(4,1) p(2,0))
    (2, 2, 1, 203, 48, 1, 8, 1, 4, 0, 2, 1, 1),     # time encoder conv
    (1, 24, 16, 11, 48, 3, 3, 1, 1, 1, 1, 1, 1),    # decoder 3x3 rewrite
    (2, 12, 1, 77, 6, 1, 3, 1, 1, 0, 2, 1, 2),      # DConv conv1, dilation 2
    (1, 5, 7, 13, 130, 1, 1, 1, 1, 0, 0, 1, 1),     # 1x1, M > 128 (two m-tiles)
    (1, 3, 9, 10, 7, 2, 3, 2, 3, 1, 2, 2, 1),       # generic kernel path
])
def test_conv2d_matches_oracle(lib, oracle, fp32_precision, b, ic, h, w, oc, kh, kw, sh, sw, ph, pw, dh, dw):
    r = rng(ic * 31 + oc)
    x = r.uniform(-0.4, 0.4, (b, ic, h, w)).astype(np.float32)
    wt = r.uniform(-0.4, 0.4, (oc, ic, kh, kw)).astype(np.float32)
    bias = r.uniform(-0.4, 0.4, oc).astype(np.float32)
    ref = oracle.conv2d(x, wt, bias, (sh, sw), (ph, pw), (dh, dw))
    out = torch.empty(ref.shape, device="cuda")
    dx, dwt, dbias = dev(x), dev(wt), dev(bias)
    call(lib, "dmx_op_conv2d", stream(), ptr(dx), None, b, ic, h, w, ptr(dwt), ptr(dbias), oc, kh, kw, sh, sw, ph,
         pw, dh, dw, 0, ptr(out))
    assert rms_relative_error(ref, out.cpu().numpy()) < 1e-5


def test_conv2d_gelu_and_skip(lib, oracle):
    r = rng(5)
    x = r.uniform(-1, 1, (2, 8, 12, 10)).astype(np.float32)
    s = r.uniform(-1, 1, x.shape).astype(np.float32)
    wt = r.uniform(-0.4, 0.4, (16, 8, 3, 3)).astype(np.float32)
    bias = r.uniform(-0.4, 0.4, 16).astype(np.float32)
    ref = oracle.gelu(oracle.conv2d(x + s, wt, bias, (1, 1), (1, 1)))
    out = torch.empty(ref.shape, device="cuda")
    dx, ds, dwt, db = dev(x), dev(s), dev(wt), dev(bias)
    call(lib, "dmx_op_conv2d", stream(), ptr(dx), ptr(ds), 2, 8, 12, 10, ptr(dwt), ptr(db), 16, 3, 3, 1, 1, 1, 1,
         1, 1, 1, ptr(out))
    assert rms_relative_error(ref, out.cpu().numpy()) < 1e-5


@pytest.mark.parametrize("b,ic,h,w,C,kh,kw", [(1, 48, 32, 12, 48, 1, 1), (2, 24, 1, 300, 24, 1, 3),
                                               (1, 16, 10, 9, 16, 3, 3), (1, 96, 4, 7, 96, 1, 1)])
def test_conv2d_glu_matches_oracle(lib, oracle, fp32_precision, b, ic, h, w, C, kh, kw):
    r = rng(C + kh)
    x = r.uniform(-0.4, 0.4, (b, ic, h, w)).astype(np.float32)
    wt = r.uniform(-0.4, 0.4, (2 * C, ic, kh, kw)).astype(np.float32)
    bias = r.uniform(-0.4, 0.4, 2 * C).astype(np.float32)
    ref = oracle.glu(oracle.conv2d(x, wt, bias, (1, 1), (kh // 2, kw // 2)))
    out = torch.empty(ref.shape, device="cuda")
    dx, dwt, db = dev(x), dev(wt), dev(bias)
    call(lib, "dmx_op_conv2d_glu", stream(), ptr(dx), None, b, ic, h, w, ptr(dwt), ptr(db), C, kh, kw, kh // 2,
         kw // 2, None, ctypes.c_float(0.0), ptr(out))
    assert rms_relative_error(ref, out.cpu().numpy()) < 1e-5


# 3x3 / padding 1 with at least 96 output channels: the decoder rewrite's
# shape, which runs as Winograd F(4x4, 3x3) (input transform, 36 batched GEMMs,
# output transform + GLU); sizes that are not multiples of 4 leave partial
# tiles at the edges.
@pytest.mark.parametrize("b,ic,h,w,C,with_skip", [(2, 192, 8, 20, 192, True), (1, 384, 8, 12, 384, True),
                                                  (1, 192, 5, 7, 192, False), (2, 208, 3, 33, 192, True),
                                                  (1, 192, 1, 1, 192, True), (2, 96, 16, 21, 96, True),
                                                  (1, 96, 32, 336, 96, True)])
def test_conv2d_glu_3x3_winograd_matches_oracle(lib, oracle, b, ic, h, w, C, with_skip):
    r = rng(ic + h * w)
    x = r.uniform(-0.4, 0.4, (b, ic, h, w)).astype(np.float32)
    skip = r.uniform(-0.4, 0.4, (b, ic, h, w)).astype(np.float32) if with_skip else np.zeros_like(x)
    wt = r.uniform(-0.1, 0.1, (2 * C, ic, 3, 3)).astype(np.float32)
    bias = r.uniform(-0.4, 0.4, 2 * C).astype(np.float32)
    ref = oracle.glu(oracle.conv2d(x + skip, wt, bias, (1, 1), (1, 1)))
    out = torch.empty(ref.shape, device="cuda")
    dx, ds, dwt, db = dev(x), dev(skip), dev(wt), dev(bias)
    call(lib, "dmx_op_conv2d_glu", stream(), ptr(dx), ptr(ds) if with_skip else None, b, ic, h, w, ptr(dwt),
         ptr(db), C, 3, 3, 1, 1, None, ctypes.c_float(0.0), ptr(out))
    assert rms_relative_error(ref, out.cpu().numpy()) < 1e-5


def test_conv2d_glu_adds_the_frequency_embedding(lib, oracle):
    r = rng(9)
    b, ic, f, t, C = 1, 48, 16, 5, 48
    x = r.uniform(-0.4, 0.4, (b, ic, f, t)).astype(np.float32)
    wt = r.uniform(-0.4, 0.4, (2 * C, ic, 1, 1)).astype(np.float32)
    bias = r.uniform(-0.4, 0.4, 2 * C).astype(np.float32)
    emb = r.normal(0, 1, (f, C)).astype(np.float32)
    ref = oracle.glu(oracle.conv2d(x, wt, bias)) + (np.float32(0.2) * emb.T)[None, :, :, None]
    out = torch.empty(ref.shape, device="cuda")
    dx, dwt, db, de = dev(x), dev(wt), dev(bias), dev(emb)
    call(lib, "dmx_op_conv2d_glu", stream(), ptr(dx), None, b, ic, f, t, ptr(dwt), ptr(db), C, 1, 1, 0, 0, ptr(de),
         ctypes.c_float(0.2), ptr(out))
    assert rms_relative_error(ref, out.cpu().numpy()) < 1e-5


@pytest.mark.parametrize("b,ic,A,P,oc,last", [(1, 48, 32, 11, 16, True), (2, 96, 8, 5, 48, False),
                                              (1, 48, 301, 1, 8, True), (2, 24, 50, 1, 12, False)])
def test_conv_transpose_matches_oracle(lib, oracle, fp32_precision, b, ic, A, P, oc, last):
    r = rng(ic + A)
    x = r.uniform(-0.4, 0.4, (b, ic, A, P)).astype(np.float32)
    wt = r.uniform(-0.4, 0.4, (ic, oc, 8, 1)).astype(np.float32)
    bias = r.uniform(-0.4, 0.4, oc).astype(np.float32)
    full = oracle.conv_transpose2d(x, wt, bias, (4, 1))
    a_out = 4 * A if P > 1 else 4 * A - 1  # the waveform crop keeps `length` <= produced - 2
    ref = full[:, :, 2:2 + a_out, :]
    if not last:
        ref = oracle.gelu(ref)
    out = torch.empty(ref.shape, device="cuda")
    dx, dw, db = dev(x), dev(wt.reshape(ic, oc, 8)), dev(bias)
    call(lib, "dmx_op_conv_transpose", stream(), ptr(dx), b, ic, A, P, ptr(dw), ptr(db), oc, 8, 4, 2, a_out,
         0 if last else 1, ptr(out))
    assert rms_relative_error(ref, out.cpu().numpy()) < 1e-5


def dconv_case(C, seed, B, F, T):
    """Random weights of a depth-2 DConv (PyTorch names under prefix "x") and
    an input (B, C, F, T), with the oracle's result for it."""
    r = rng(seed)
    hid = C // 8
    w = {}
    for d in range(2):
        at = f"x.layers.{d}"
        w[f"{at}.0.weight"] = r.uniform(-0.5, 0.5, (hid, C, 3)).astype(np.float32)
        w[f"{at}.0.bias"] = r.uniform(-0.3, 0.3, hid).astype(np.float32)
        w[f"{at}.1.weight"] = r.uniform(0.75, 1.25, hid).astype(np.float32)
        w[f"{at}.1.bias"] = r.uniform(-0.2, 0.2, hid).astype(np.float32)
        w[f"{at}.3.weight"] = r.uniform(-0.5, 0.5, (2 * C, hid, 1)).astype(np.float32)
        w[f"{at}.3.bias"] = r.uniform(-0.3, 0.3, 2 * C).astype(np.float32)
        w[f"{at}.4.weight"] = r.uniform(0.75, 1.25, 2 * C).astype(np.float32)
        w[f"{at}.4.bias"] = r.uniform(-0.2, 0.2, 2 * C).astype(np.float32)
        w[f"{at}.6.scale"] = r.uniform(0.1, 0.5, C).astype(np.float32)
    x = r.uniform(-1, 1, (B, C, F, T)).astype(np.float32)
    return hid, w, x


DCONV_PARAMS = ("0.weight", "0.bias", "1.weight", "1.bias", "3.weight", "3.bias", "4.weight", "4.bias", "6.scale")


def dconv_reference(oracle, x, w):
    B, C, F, T = x.shape
    rows = x.transpose(0, 2, 1, 3).reshape(B * F, C, T)
    return oracle.dconv(rows, w, "x").reshape(B, F, C, T).transpose(0, 2, 1, 3)


@pytest.mark.parametrize("B,C,F,T", [(1, 48, 16, 40), (2, 96, 1, 700), (1, 384, 2, 33), (2, 192, 3, 300),
                                     (1, 48, 1, 1000), (2, 48, 3, 77), (1, 96, 5, 65), (1, 96, 2, 336),
                                     (1, 192, 1, 1500), (1, 384, 2, 336)])
def test_dconv_matches_oracle(lib, oracle, fp32_precision, dmx, B, C, F, T):
    hid, w, x = dconv_case(C, C + T, B, F, T)
    ref = dconv_reference(oracle, x, w)
    dx = dev(x)
    dw = {k: dev(v) for k, v in w.items()}
    for d in range(2):
        at = f"x.layers.{d}"
        call(lib, "dmx_op_dconv_layer", stream(), ptr(dx), B, C, F, T, 1 << d, ptr(dw[f"{at}.0.weight"]),
             ptr(dw[f"{at}.0.bias"]), hid, ptr(dw[f"{at}.1.weight"]), ptr(dw[f"{at}.1.bias"]),
             ptr(dw[f"{at}.3.weight"]), ptr(dw[f"{at}.3.bias"]), ptr(dw[f"{at}.4.weight"]), ptr(dw[f"{at}.4.bias"]),
             ptr(dw[f"{at}.6.scale"]))
    assert rms_relative_error(ref, dx.cpu().numpy()) < 1e-5


# Rows of up to 384 positions at C = 48 / 96 run both layers in one launch
# with the row in LDS (T = 336 is the spectral branch's row); the others take
# the per-layer path behind the same entry point.
@pytest.mark.parametrize("B,C,F,T", [(2, 96, 4, 336), (1, 48, 8, 336), (1, 48, 16, 40), (3, 48, 2, 1),
                                     (1, 96, 3, 384), (2, 48, 3, 77), (1, 96, 5, 65), (1, 48, 2, 385),
                                     (2, 96, 1, 700), (1, 192, 2, 50)])
def test_dconv_both_layers_matches_oracle(lib, oracle, dmx, B, C, F, T):
    hid, w, x = dconv_case(C, 7 * C + T, B, F, T)
    ref = dconv_reference(oracle, x, w)
    dx = dev(x)
    dw = [dev(w[f"x.layers.{d}.{name}"]) for d in range(2) for name in DCONV_PARAMS]
    params = (ctypes.c_void_p * 18)(*[t.data_ptr() for t in dw])
    call(lib, "dmx_op_dconv", stream(), ptr(dx), B, C, F, T, hid, params)
    assert rms_relative_error(ref, dx.cpu().numpy()) < 1e-5


# Key counts cover one to five 32-key tiles, whole and ragged, so the
# three-plane kernel's pipelined loop runs with odd and even tile counts.
@pytest.mark.parametrize("batch,heads,nq,nk", [(1, 8, 200, 130), (2, 2, 64, 64), (1, 1, 33, 1), (1, 8, 2688, 1344),
                                               (1, 2, 50, 32), (1, 2, 40, 40), (1, 2, 70, 96), (2, 1, 65, 128)])
def test_attention_matches_oracle(lib, oracle, fp32_precision, batch, heads, nq, nk):
    r = rng(nq + nk)
    D = heads * 64
    q = r.uniform(-2, 2, (batch, nq, D)).astype(np.float32)
    k = r.uniform(-2, 2, (batch, nk, D)).astype(np.float32)
    v = r.uniform(-2, 2, (batch, nk, D)).astype(np.float32)
    ref = np.empty_like(q)
    for b in range(batch):
        for h in range(heads):
            sl = slice(64 * h, 64 * h + 64)
            ref[b, :, sl] = oracle.attention_head(q[b, :, sl], k[b, :, sl], v[b, :, sl], 0.125)
    out = torch.empty(q.shape, device="cuda")
    dq, dk, dv = dev(q), dev(k), dev(v)
    call(lib, "dmx_op_attention", stream(), ptr(dq), ptr(dk), ptr(dv), ptr(out), batch, heads, nq, nk,
         ctypes.c_float(0.125))
    assert rms_relative_error(ref, out.cpu().numpy()) < 1e-5


@pytest.mark.parametrize("batch,heads,nq0,nk0,nq1,nk1", [(2, 2, 200, 70, 70, 200), (1, 8, 2688, 1344, 1344, 2688),
                                                        (3, 1, 33, 5, 129, 129)])
def test_attention_pair_matches_oracle(lib, oracle, fp32_precision, batch, heads, nq0, nk0, nq1, nk1):
    """Two problems in one launch (the blocks of the one with more keys come
    first): each output matches the oracle on its own problem."""
    r = rng(nq0 + 7 * nk1)
    D = heads * 64
    probs = []
    for nq, nk in ((nq0, nk0), (nq1, nk1)):
        q = r.uniform(-2, 2, (batch, nq, D)).astype(np.float32)
        k = r.uniform(-2, 2, (batch, nk, D)).astype(np.float32)
        v = r.uniform(-2, 2, (batch, nk, D)).astype(np.float32)
        ref = np.empty_like(q)
        for b in range(batch):
            for h in range(heads):
                sl = slice(64 * h, 64 * h + 64)
                ref[b, :, sl] = oracle.attention_head(q[b, :, sl], k[b, :, sl], v[b, :, sl], 0.125)
        probs.append((dev(q), dev(k), dev(v), torch.empty(q.shape, device="cuda"), ref, nq, nk))
    (q0, k0, v0, o0, r0, _, _), (q1, k1, v1, o1, r1, _, _) = probs
    call(lib, "dmx_op_attention_pair", stream(), ptr(q0), ptr(k0), ptr(v0), ptr(o0), nq0, nk0, ptr(q1), ptr(k1),
         ptr(v1), ptr(o1), nq1, nk1, batch, heads, ctypes.c_float(0.125))
    assert rms_relative_error(r0, o0.cpu().numpy()) < 1e-5
    assert rms_relative_error(r1, o1.cpu().numpy()) < 1e-5


@pytest.mark.parametrize("ramp", [1.0, 3.0, -3.0])
def test_attention_running_max_moves_across_tiles(lib, oracle, fp32_precision, ramp):
    """Key norms ramp along the sequence, so each query's row max keeps rising
    (or falls after the first tile) by many times 2^8 in probability: every
    rescale path of the online softmax runs, and the last tile is ragged."""
    r = rng(77)
    nq, nk, heads = 150, 700, 2
    D = heads * 64
    q = r.uniform(-2, 2, (1, nq, D)).astype(np.float32)
    gain = np.exp(ramp * np.linspace(0.0, 1.0, nk, dtype=np.float32))[None, :, None]
    k = (r.uniform(-2, 2, (1, nk, D)) * gain).astype(np.float32)
    v = r.uniform(-2, 2, (1, nk, D)).astype(np.float32)
    ref = np.empty_like(q)
    for h in range(heads):
        sl = slice(64 * h, 64 * h + 64)
        ref[0, :, sl] = oracle.attention_head(q[0, :, sl], k[0, :, sl], v[0, :, sl], 0.125)
    out = torch.empty(q.shape, device="cuda")
    dq, dk, dv = dev(q), dev(k), dev(v)
    call(lib, "dmx_op_attention", stream(), ptr(dq), ptr(dk), ptr(dv), ptr(out), 1, heads, nq, nk,
         ctypes.c_float(0.125))
    assert rms_relative_error(ref, out.cpu().numpy()) < 1e-5


@pytest.mark.parametrize("rows,dim", [(333, 512), (77, 100)])  # the float4 register path, the generic one
def test_layer_norm_matches_oracle(lib, oracle, rows, dim):
    r = rng(1)
    x = r.uniform(-3, 3, (rows, dim)).astype(np.float32)
    w, b = r.uniform(0.5, 1.5, dim).astype(np.float32), r.uniform(-1, 1, dim).astype(np.float32)
    ref = oracle.layer_norm(x, w, b)
    out = torch.empty(x.shape, device="cuda")
    dx, dw, db = dev(x), dev(w), dev(b)
    call(lib, "dmx_op_layer_norm", stream(), ptr(dx), rows, dim, ptr(dw), ptr(db), ptr(out))
    assert rms_relative_error(ref, out.cpu().numpy()) < 1e-6


@pytest.mark.parametrize("b,c,inner,groups", [(2, 8, 1000, 1), (1, 16, 77, 4), (3, 6, 5, 2)])
def test_group_norm_matches_oracle(lib, oracle, b, c, inner, groups):
    r = rng(c * inner)
    x = r.uniform(-3, 3, (b, c, inner)).astype(np.float32)
    w, bias = r.uniform(0.5, 1.5, c).astype(np.float32), r.uniform(-1, 1, c).astype(np.float32)
    ref = oracle.group_norm(x, groups, w, bias)
    out = torch.empty(x.shape, device="cuda")
    dx, dw, db = dev(x), dev(w), dev(bias)
    call(lib, "dmx_op_group_norm", stream(), ptr(dx), b, c, inner, groups, ptr(dw), ptr(db), ptr(out))
    assert rms_relative_error(ref, out.cpu().numpy()) < 1e-6


def test_glu_and_gelu_match_oracle(lib, oracle):
    r = rng(2)
    x = r.uniform(-6, 6, (2, 10, 333)).astype(np.float32)
    ref_glu, ref_gelu = oracle.glu(x), oracle.gelu(x)
    out = torch.empty(ref_glu.shape, device="cuda")
    out2 = torch.empty(x.shape, device="cuda")
    dx = dev(x)
    call(lib, "dmx_op_glu", stream(), ptr(dx), 2, 10, 333, ptr(out))
    call(lib, "dmx_op_gelu", stream(), ptr(dx), x.size, ptr(out2))
    assert rms_relative_error(ref_glu, out.cpu().numpy()) < 1e-6
    assert rms_relative_error(ref_gelu, out2.cpu().numpy()) < 1e-6


@pytest.mark.parametrize("b,L", [(1, 11025), (2, 30000)])
def test_spec_normalise_matches_oracle(lib, oracle, b, L):
    r = rng(L)
    mix = r.normal(0, 0.1, (b, 2, L)).astype(np.float32)
    spec = oracle.spec_cac(mix)
    xs_ref = np.empty_like(spec)
    xt_ref = np.empty_like(mix)
    norms_ref = np.empty((b, 4), np.float32)
    for i in range(b):
        m, s = oracle.mean(spec[i]), oracle.std_unbiased(spec[i])
        mt, st = oracle.mean(mix[i]), oracle.std_unbiased(mix[i])
        xs_ref[i] = (spec[i] - np.float32(m)) * np.float32(1.0 / (1e-5 + np.float32(s)))
        xt_ref[i] = (mix[i] - np.float32(mt)) * np.float32(1.0 / (1e-5 + np.float32(st)))
        norms_ref[i] = (m, s, mt, st)
    xs = torch.empty(spec.shape, device="cuda")
    xt = torch.empty(mix.shape, device="cuda")
    norms = torch.empty((b, 4), device="cuda")
    dmix = dev(mix)
    call(lib, "dmx_op_spec_normalise", stream(), ptr(dmix), b, L, ptr(xs), ptr(xt), ptr(norms))
    np.testing.assert_allclose(norms.cpu().numpy(), norms_ref, rtol=1e-5, atol=1e-7)
    assert snr_db(xs_ref, xs.cpu().numpy()) > 100  # f32 FFT against the f64 oracle FFT
    assert rms_relative_error(xt_ref, xt.cpu().numpy()) < 1e-6


@pytest.mark.parametrize("b,L", [(1, 11025), (2, 30000)])
def test_ispec_sum_matches_oracle(lib, oracle, b, L):
    r = rng(L + 1)
    le = -(-L // 1024)
    xs = r.normal(0, 1, (b, 16, 2048, le)).astype(np.float32)
    xt = r.normal(0, 1, (b, 8, L)).astype(np.float32)
    norms = np.array([[0.01 * (i + 1), 0.5 + i, -0.02, 0.3] for i in range(b)], np.float32)
    ref = np.empty((b, 4, 2, L), np.float32)
    for i in range(b):
        m, s, mt, st = norms[i]
        den = (xs[i:i + 1] - np.float32(-m / s)) * np.float32(s)
        wave = oracle.ispec_cac(den, 4, L)
        tim = ((xt[i] - np.float32(-mt / st)) * np.float32(st)).reshape(4, 2, L)
        ref[i] = tim + wave[0]
    out = torch.empty(ref.shape, device="cuda")
    dxs, dxt, dn = dev(xs), dev(xt), dev(norms)
    call(lib, "dmx_op_ispec_sum", stream(), ptr(dxs), ptr(dxt), b, L, ptr(dn), ptr(out))
    assert snr_db(ref, out.cpu().numpy()) > 100


@pytest.mark.parametrize("rows,k,n", [(2688, 512, 1536), (1344, 2048, 512), (200, 512, 2048)])
def test_plane_linear_is_fp32_accurate(lib, rows, k, n):
    """The three-plane product keeps fp32 accuracy: against a float64
    reference its worst error is no larger than twice that of the fp32-MFMA
    kernel on the same operands, and far below a one-plane (bf16) product's.
    Operands span 2^-20 .. 2^4 in magnitude so that the low planes matter."""
    r = rng(rows * 3 + k + n)
    x = (r.standard_normal((rows, k)) * np.exp2(r.uniform(-20, 4, (rows, k)))).astype(np.float32)
    w = (r.standard_normal((n, k)) * np.exp2(r.uniform(-8, 0, (n, k)))).astype(np.float32)
    b = np.zeros(n, np.float32)
    ref = x.astype(np.float64) @ w.T.astype(np.float64)
    dx, dw, db = dev(x), dev(w), dev(b)
    errs = {}
    for prec in (0, 2, 1):
        assert lib.dmx_op_set_precision(prec) == 0
        out = torch.empty((rows, n), device="cuda")
        call(lib, "dmx_op_linear", stream(), ptr(dx), rows, k, ptr(dw), ptr(db), n, 0, None, None, ptr(out))
        errs[prec] = float(np.abs(out.cpu().numpy().astype(np.float64) - ref).max())
    assert lib.dmx_op_set_precision(0) == 0
    scale = float(np.abs(ref).max())
    assert errs[0] <= 2.0 * errs[2] + 1e-7 * scale, errs
    assert errs[0] < 1e-2 * errs[1], errs


@pytest.mark.parametrize("nk0,nk1", [(1344, 2688), (70, 333)])
def test_attention_pair_on_kv_planes_matches_pair(lib, nk0, nk1):
    """dmx_op_kv_planes + dmx_op_attention_pair_planes (the launch bench.py
    times) give what dmx_op_attention_pair gives under the default precision,
    bit for bit: the same kernel on the same planes."""
    r = rng(nk0 + nk1)
    batch, heads = 2, 2
    D = heads * 64
    nq0, nq1 = nk1, nk0
    q0, q1 = (dev(r.uniform(-2, 2, (batch, n, D)).astype(np.float32)) for n in (nq0, nq1))
    k0, v0 = (dev(r.uniform(-2, 2, (batch, nk0, D)).astype(np.float32)) for _ in range(2))
    k1, v1 = (dev(r.uniform(-2, 2, (batch, nk1, D)).astype(np.float32)) for _ in range(2))
    ref0, ref1 = torch.empty(batch, nq0, D, device="cuda"), torch.empty(batch, nq1, D, device="cuda")
    assert lib.dmx_op_set_precision(0) == 0
    call(lib, "dmx_op_attention_pair", stream(), ptr(q0), ptr(k0), ptr(v0), ptr(ref0), nq0, nk0, ptr(q1), ptr(k1),
         ptr(v1), ptr(ref1), nq1, nk1, batch, heads, ctypes.c_float(0.125))
    planes = []
    for k, v, nk in ((k0, v0, nk0), (k1, v1, nk1)):
        ldvt = (nk + 31) // 32 * 32
        kp = torch.empty(3 * batch * nk * D, dtype=torch.int16, device="cuda")
        vt = torch.empty(3 * batch * D * ldvt, dtype=torch.int16, device="cuda")
        call(lib, "dmx_op_kv_planes", stream(), ptr(k), ptr(v), batch, heads, nk, ptr(kp), ptr(vt))
        planes.append((kp, vt))
    o0, o1 = torch.empty_like(ref0), torch.empty_like(ref1)
    call(lib, "dmx_op_attention_pair_planes", stream(), ptr(q0), ptr(planes[0][0]), ptr(planes[0][1]), ptr(o0), nq0,
         nk0, ptr(q1), ptr(planes[1][0]), ptr(planes[1][1]), ptr(o1), nq1, nk1, batch, heads, ctypes.c_float(0.125))
    torch.cuda.synchronize()
    assert torch.equal(o0, ref0) and torch.equal(o1, ref1)


@pytest.mark.parametrize("nq,nk", [(2688, 1344), (1344, 2688), (300, 333)])
def test_plane_attention_is_fp32_accurate(lib, nq, nk):
    """The three-plane attention keeps fp32 accuracy: against a float64
    softmax its worst error is at most twice the fp32-MFMA kernel's, and far
    below the bf16 kernel's."""
    r = rng(nq + 3 * nk)
    heads, D = 2, 128
    q = r.uniform(-2, 2, (1, nq, D)).astype(np.float32)
    k = r.uniform(-2, 2, (1, nk, D)).astype(np.float32)
    v = r.uniform(-2, 2, (1, nk, D)).astype(np.float32)
    ref = np.empty(q.shape, np.float64)
    for h in range(heads):
        sl = slice(64 * h, 64 * h + 64)
        s_ = (q[0, :, sl].astype(np.float64) * 0.125) @ k[0, :, sl].astype(np.float64).T
        p_ = np.exp(s_ - s_.max(axis=1, keepdims=True))
        ref[0, :, sl] = (p_ @ v[0, :, sl].astype(np.float64)) / p_.sum(axis=1, keepdims=True)
    dq, dk, dv = dev(q), dev(k), dev(v)
    errs = {}
    for prec in (0, 2, 1):
        assert lib.dmx_op_set_precision(prec) == 0
        out = torch.empty(q.shape, device="cuda")
        call(lib, "dmx_op_attention", stream(), ptr(dq), ptr(dk), ptr(dv), ptr(out), 1, heads, nq, nk,
             ctypes.c_float(0.125))
        errs[prec] = float(np.abs(out.cpu().numpy().astype(np.float64) - ref).max())
    assert lib.dmx_op_set_precision(0) == 0
    assert errs[0] <= 2.0 * errs[2] + 1e-7, errs
    assert errs[0] < 1e-2 * errs[1], errs


# ---- bf16-MFMA variant: inputs rounded to bf16, fp32 accumulation and output.
# Gate: rms-relative error <= 1e-2 against the fp32 oracle (bf16 keeps 8
# mantissa bits, 2^-9 relative rounding per operand), and > 1e-5 so the test
# proves the bf16 kernel ran rather than the fp32 one.

@pytest.fixture
def bf16(lib):
    assert lib.dmx_op_set_precision(1) == 0
    yield
    assert lib.dmx_op_set_precision(0) == 0


def test_bf16_precision_is_validated(lib):
    assert lib.dmx_op_set_precision(7) != 0
    assert lib.dmx_op_set_precision(0) == 0


@pytest.mark.parametrize("rows,k,n,tail", [(300, 512, 1536, 0), (64, 512, 2048, 1), (129, 2048, 512, 2),
                                           (37, 19, 70, 0)])
def test_bf16_linear_matches_oracle(lib, oracle, bf16, rows, k, n, tail):
    r = rng(rows + k + n + 1)
    x = r.uniform(-0.4, 0.4, (rows, k)).astype(np.float32)
    w = r.uniform(-0.4, 0.4, (n, k)).astype(np.float32)
    b = r.uniform(-0.4, 0.4, n).astype(np.float32)
    res = r.uniform(-1, 1, (rows, n)).astype(np.float32)
    g = r.uniform(0.1, 0.5, n).astype(np.float32)
    ref = oracle.sgemm(x, w.T) + b
    if tail == 1:
        ref = oracle.gelu(ref)
    elif tail == 2:
        ref = res + ref * g
    dx, dw, db, dres, dg = dev(x), dev(w), dev(b), dev(res), dev(g)
    out = torch.empty((rows, n), device="cuda")
    call(lib, "dmx_op_linear", stream(), ptr(dx), rows, k, ptr(dw), ptr(db), n, tail, ptr(dres), ptr(dg), ptr(out))
    err = rms_relative_error(ref, out.cpu().numpy())
    assert 1e-5 < err < 1e-2, err


@pytest.mark.parametrize("b,ic,h,w,C,kh,kw", [(1, 48, 32, 12, 48, 1, 1), (1, 16, 10, 9, 16, 3, 3),
                                               (2, 24, 1, 300, 24, 1, 3)])
def test_bf16_conv2d_glu_matches_oracle(lib, oracle, bf16, b, ic, h, w, C, kh, kw):
    r = rng(C + kh + 1)
    x = r.uniform(-0.4, 0.4, (b, ic, h, w)).astype(np.float32)
    wt = r.uniform(-0.4, 0.4, (2 * C, ic, kh, kw)).astype(np.float32)
    bias = r.uniform(-0.4, 0.4, 2 * C).astype(np.float32)
    ref = oracle.glu(oracle.conv2d(x, wt, bias, (1, 1), (kh // 2, kw // 2)))
    out = torch.empty(ref.shape, device="cuda")
    dx, dwt, db = dev(x), dev(wt), dev(bias)
    call(lib, "dmx_op_conv2d_glu", stream(), ptr(dx), None, b, ic, h, w, ptr(dwt), ptr(db), C, kh, kw, kh // 2,
         kw // 2, None, ctypes.c_float(0.0), ptr(out))
    err = rms_relative_error(ref, out.cpu().numpy())
    assert 1e-5 < err < 1e-2, err


@pytest.mark.parametrize("batch,heads,nq,nk", [(1, 8, 200, 130), (1, 1, 33, 1), (2, 8, 2688, 1344)])
def test_bf16_attention_matches_oracle(lib, oracle, bf16, batch, heads, nq, nk):
    r = rng(nq + nk + 1)
    D = heads * 64
    q = r.uniform(-2, 2, (batch, nq, D)).astype(np.float32)
    k = r.uniform(-2, 2, (batch, nk, D)).astype(np.float32)
    v = r.uniform(-2, 2, (batch, nk, D)).astype(np.float32)
    ref = np.empty_like(q)
    for bb in range(batch):
        for h in range(heads):
            sl = slice(64 * h, 64 * h + 64)
            ref[bb, :, sl] = oracle.attention_head(q[bb, :, sl], k[bb, :, sl], v[bb, :, sl], 0.125)
    out = torch.empty(q.shape, device="cuda")
    dq, dk, dv = dev(q), dev(k), dev(v)
    call(lib, "dmx_op_attention", stream(), ptr(dq), ptr(dk), ptr(dv), ptr(out), batch, heads, nq, nk,
         ctypes.c_float(0.125))
    err = rms_relative_error(ref, out.cpu().numpy())
    assert (nk == 1 or 1e-5 < err) and err < 1e-2, err
