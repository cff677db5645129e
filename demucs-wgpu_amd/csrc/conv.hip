// conv.hip — every GEMM-shaped op of the forward, as loaders + epilogues over
// the MFMA GEMM of gemm.h: implicit-GEMM convolutions (nothing im2col'd to
// HBM), GLU-fused rewrites, transposed convolutions as per-phase GEMMs, the
// fused DConv layer, channel mixers and the transformer linears.
#include <cstdlib>
#include <type_traits>

#include "gemm.h"
#include "gemm_planes.h"
#include "ops.h"

namespace dmx {
namespace {

// ---------------------------------------------------------------------------
// Loaders
// ---------------------------------------------------------------------------

// Implicit im2col of nn.Conv2d (crates/demucs-core/src/demucs/ops.rs:44-211):
// B[k][n] with k = (ic, ky, kx), n = (oy, ox); zero outside the input.
// The z-th problem's input starts at (z / zdiv) * outer + (z % zdiv) * inner,
// which lets a DConv treat the (b, f) rows of a (B, C, F, T) tensor as its
// batch without a permute. KH/KW > 0 fix the kernel at compile time.
template <int KH, int KW>
struct ConvGather {
    static constexpr bool kmajor = false;
    __device__ bool fast() const { return true; }
    const float *x, *skip;
    int64_t outer, inner, cs;  // batch strides and channel stride
    int zdiv, h, w, kh_rt, kw_rt, sh, sw, ph, pw, dh, dw, ow;
    struct State {
        const float *base;
        const float *sbase;
        int iy0, ix0;
    };
    __device__ int kh() const { return KH > 0 ? KH : kh_rt; }
    __device__ int kw() const { return KW > 0 ? KW : kw_rt; }
    __device__ State setup(int z, int n) const {
        int oy = n / ow, ox = n - oy * ow;
        int64_t off = (int64_t)(z / zdiv) * outer + (int64_t)(z % zdiv) * inner;
        return {x + off, skip ? skip + off : nullptr, oy * sh - ph, ox * sw - pw};
    }
    __device__ float load(const State &s, int k) const {
        const int taps = kh() * kw();
        int c = k / taps, tap = k - c * taps;
        int ky = tap / kw(), kx = tap - ky * kw();
        int iy = s.iy0 + ky * dh, ix = s.ix0 + kx * dw;
        if (iy < 0 || iy >= h || ix < 0 || ix >= w) return 0.0f;
        int64_t at = c * cs + (int64_t)iy * w + ix;
        float v = s.base[at];
        if (s.sbase) v += s.sbase[at];
        return v;
    }
};

// The same gather in channel-quad order: k = (c / 4 * taps + tap) * 4 + c % 4,
// matching weights in GEMM order (conv_tap_major). The four k of a quad are
// four channels at one tap: one bounds test, then four loads one channel
// stride apart; the taps of a quad are adjacent in k, so the input rows of
// one k-tile are mostly the previous tile's (cache hits). SKIP adds the skip
// tensor in finish(), after the k-tile's MFMAs.
template <int KH, int KW, bool SKIP>
struct ConvGatherTM {
    static constexpr bool kmajor = false;
    __device__ bool fast() const { return true; }
    const float *x, *skip;
    int64_t outer, inner, cs;  // batch strides and channel stride
    int zdiv, h, w, sh, sw, ph, pw, dh, dw, ow, kh_rt, kw_rt;
    using State = typename ConvGather<KH, KW>::State;
    struct Raw {
        float4 x, s;
    };
    __device__ int kw() const { return KW > 0 ? KW : kw_rt; }
    __device__ int taps() const { return KH > 0 && KW > 0 ? KH * KW : kh_rt * kw_rt; }
    __device__ State setup(int z, int n) const {
        int oy = n / ow, ox = n - oy * ow;
        int64_t off = (int64_t)(z / zdiv) * outer + (int64_t)(z % zdiv) * inner;
        return {x + off, SKIP ? skip + off : nullptr, oy * sh - ph, ox * sw - pw};
    }
    __device__ Raw zero_raw() const {
        const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
        return {z, z};
    }
    __device__ Raw load_raw(const State &s, int k) const {
        const int q = k >> 2, cq = q / taps(), tap = q - cq * taps();
        const int ky = tap / kw(), kx = tap - ky * kw();
        const int iy = s.iy0 + ky * dh, ix = s.ix0 + kx * dw;
        if (iy < 0 || iy >= h || ix < 0 || ix >= w) return zero_raw();
        const int64_t at = 4 * cq * cs + (int64_t)iy * w + ix;
        const float *p = s.base + at;
        Raw r;
        r.x = make_float4(p[0], p[cs], p[2 * cs], p[3 * cs]);
        if constexpr (SKIP) {
            const float *q2 = s.sbase + at;
            r.s = make_float4(q2[0], q2[cs], q2[2 * cs], q2[3 * cs]);
        }
        return r;
    }
    __device__ float4 finish(const State &, const Raw &r, int) const {
        if constexpr (SKIP)
            return make_float4(r.x.x + r.s.x, r.x.y + r.s.y, r.x.z + r.s.z, r.x.w + r.s.w);
        else
            return r.x;
    }
};

// DConv conv2's input: GroupNorm(1) + GELU of conv1's output, applied while
// loading. y is (rows, H, T); stats holds (sum, sum_sq) per row.
struct NormGeluRows {
    static constexpr bool kmajor = false;
    __device__ bool fast() const { return true; }
    const float *y;
    const double *stats;
    const float *nw, *nb;
    int H, T;
    struct State {
        const float *col;
        float mean, inv;
    };
    __device__ State setup(int z, int n) const {
        float mean, inv;
        gn_stats(stats + 2 * z, (double)H * (double)T, mean, inv);
        return {y + (int64_t)z * H * T + n, mean, inv};
    }
    __device__ float load(const State &s, int k) const {
        float scale = s.inv * nw[k];
        float shift = nb[k] - s.mean * scale;
        return gelu(s.col[(int64_t)k * T] * scale + shift);
    }
};

// NormGeluRows for H % 4 == 0, split in two: load_raw fetches four hidden
// rows of the column before the k-tile's MFMAs, finish applies GN + GELU
// after them (k >= H finishes to zero).
struct NormGeluQuads {
    static constexpr bool kmajor = false;
    __device__ bool fast() const { return true; }
    const float *y;
    const double *stats;
    const float *nw, *nb;
    int H, T;
    using State = NormGeluRows::State;
    using Raw = float4;
    __device__ State setup(int z, int n) const {
        float mean, inv;
        gn_stats(stats + 2 * z, (double)H * (double)T, mean, inv);
        return {y + (int64_t)z * H * T + n, mean, inv};
    }
    __device__ Raw zero_raw() const { return make_float4(0.f, 0.f, 0.f, 0.f); }
    __device__ Raw load_raw(const State &s, int k) const {
        const float *p = s.col + (int64_t)k * T;
        return make_float4(p[0], p[T], p[2 * (int64_t)T], p[3 * (int64_t)T]);
    }
    __device__ float4 finish(const State &s, const Raw &r, int k) const {
        if (k >= H) return make_float4(0.f, 0.f, 0.f, 0.f);
        auto one = [&](float v, int kk) {
            const float scale = s.inv * nw[kk];
            return gelu(v * scale + (nb[kk] - s.mean * scale));
        };
        return make_float4(one(r.x, k), one(r.y, k + 1), one(r.z, k + 2), one(r.w, k + 3));
    }
};

// Rows of the DConv hidden activation g = GELU(GN1(y)) along t, k-major, for
// the Gram matrix G = g g^T: batch z is (row z / chunks, t-chunk z % chunks)
// of `chunk` positions; logical row H is a row of ones (its products give
// the per-channel sums of g), rows past it and positions past T read zero.
struct GramRows {
    static constexpr bool kmajor = true;
    const float *y;
    const double *stats;
    const float *nw, *nb;
    int H, T, chunk, chunks;
    struct State {
        const float *row;  // first position of the chunk, or null for the ones row
        float scale, shift;
        int valid;         // positions of this chunk inside the row
        bool ones;
    };
    __device__ bool fast() const { return false; }
    __device__ State setup(int z, int r) const {
        const int row = z / chunks, t0 = (z - row * chunks) * chunk;
        const int valid = min(chunk, T - t0);
        if (r >= H) return {nullptr, 0.f, 0.f, r == H ? valid : 0, true};
        float mean, inv;
        gn_stats(stats + 2 * row, (double)H * (double)T, mean, inv);
        const float sc = inv * nw[r];
        return {y + ((int64_t)row * H + r) * T + t0, sc, nb[r] - mean * sc, valid, false};
    }
    __device__ float one(const State &s, int k) const {
        if (k >= s.valid) return 0.f;
        return s.ones ? 1.f : gelu(s.row[k] * s.scale + s.shift);
    }
    __device__ float4 load4_full(const State &st, int k) const { return load4(st, k, 0); }
    __device__ float4 load4(const State &st, int k, int) const {
        if (!st.ones && k + 3 < st.valid && ((reinterpret_cast<uintptr_t>(st.row + k) & 15) == 0)) {
            const float4 v = *reinterpret_cast<const float4 *>(st.row + k);
            return make_float4(gelu(v.x * st.scale + st.shift), gelu(v.y * st.scale + st.shift),
                               gelu(v.z * st.scale + st.shift), gelu(v.w * st.scale + st.shift));
        }
        return make_float4(one(st, k), one(st, k + 1), one(st, k + 2), one(st, k + 3));
    }
};

// Transposed convolution (kernel = 2 * stride) along one axis, every output
// phase in one GEMM: B[k][n] with k = 2 c + j (input channel c, tap j) and
// column n = qi * P + t is x[b][c][q - j][t] with q = q0 + qi, zero outside
// [0, A). Each input value then feeds 2 k-rows (its two taps) instead of one
// per (phase, tap) pair. A quad of k is two channels x two taps.
struct ConvTGather {
    static constexpr bool kmajor = false;
    __device__ bool fast() const { return true; }
    const float *x;
    int ic, A, P, q0;
    struct State {
        const float *base;
        int q;
    };
    __device__ State setup(int z, int n) const {
        const int qi = n / P, t = n - qi * P;
        return {x + (int64_t)z * ic * A * P + t, q0 + qi};
    }
    __device__ float4 load_quad(const State &s, int k) const {
        const int c = k >> 1;
        const bool in0 = s.q >= 0 && s.q < A, in1 = s.q >= 1 && s.q - 1 < A;
        const float *p0 = s.base + ((int64_t)c * A + s.q) * P;  // channel c, row q
        const int64_t cstride = (int64_t)A * P;
        float4 v;
        v.x = in0 ? p0[0] : 0.f;
        v.y = in1 ? p0[-P] : 0.f;
        v.z = in0 ? p0[cstride] : 0.f;
        v.w = in1 ? p0[cstride - P] : 0.f;
        return v;
    }
};

// Phase-packed transposed-conv weights (st, oc, ic*taps), read as the rows
// m = o * st + p (output channel o, phase p) of one (oc * st, ic * taps)
// matrix; k-major rows.
struct PhaseWeights {
    static constexpr bool kmajor = true;
    const float *w;
    int st, oc, K;
    bool vec;
    struct State {
        const float *row;
    };
    __device__ State setup(int, int m) const {
        const int o = m / st, p = m - o * st;
        return {w + ((int64_t)p * oc + o) * K};
    }
    __device__ bool fast() const { return vec; }
    __device__ float4 load4_full(const State &s, int k) const { return *reinterpret_cast<const float4 *>(s.row + k); }
    __device__ float4 load4(const State &s, int k, int Kt) const {
        if (vec && k + 3 < Kt) return *reinterpret_cast<const float4 *>(s.row + k);
        float4 v;
        v.x = k < Kt ? s.row[k] : 0.f;
        v.y = k + 1 < Kt ? s.row[k + 1] : 0.f;
        v.z = k + 2 < Kt ? s.row[k + 2] : 0.f;
        v.w = k + 3 < Kt ? s.row[k + 3] : 0.f;
        return v;
    }
};

// Transformer tokens (b, T*F, D) read as a (D, F*T) channel-major operand:
// column n = f*T + t is token t*F + f.
struct TokenGather {
    static constexpr bool kmajor = true;
    const float *tok;
    int F, T, D;
    struct State {
        const float *row;
    };
    __device__ State setup(int z, int n) const {
        int f = n / T, t = n - f * T;
        return {tok + ((int64_t)z * F * T + (int64_t)t * F + f) * D};
    }
    __device__ bool fast() const { return true; }  // the launcher requires D % 4 == 0 and aligned rows
    __device__ float4 load4_full(const State &s, int k) const { return *reinterpret_cast<const float4 *>(s.row + k); }
    __device__ float4 load4(const State &s, int k, int K) const {
        if (k + 3 < K) return *reinterpret_cast<const float4 *>(s.row + k);
        float4 v;
        v.x = k < K ? s.row[k] : 0.f;
        v.y = k + 1 < K ? s.row[k + 1] : 0.f;
        v.z = k + 2 < K ? s.row[k + 2] : 0.f;
        v.w = k + 3 < K ? s.row[k + 3] : 0.f;
        return v;
    }
};

// ---------------------------------------------------------------------------
// Epilogues
// ---------------------------------------------------------------------------

__device__ __forceinline__ float act_apply(int act, float v) { return act == ACT_GELU ? gelu(v) : v; }

// out[z][m][n] = act(v + bias[m]), row length N.
struct EpChannels : EpBase {
    float *out;
    const float *bias;
    int64_t batch_stride;
    int N, act;
    bool vec;  // bias null or 16-byte aligned: store_frags may read float4 biases
    __device__ void store(int z, int m, int n, float v) {
        float b = bias ? bias[m] : 0.0f;
        out[z * batch_stride + (int64_t)m * N + n] = act_apply(act, v + b);
    }
    // Whole fragments: register r of fragment (i, j) is row mb + 32 i + 8 (r / 4)
    // + 4 khalf + r % 4, so each run of four registers takes one float4 of
    // biases (mb is a multiple of 4).
    static constexpr bool frags = true;
    template <int TM, int TN>
    __device__ void store_frags(int z, int mb, int nb, int col, int khalf, const floatx16 (&v)[TM][TN]) {
        float *zo = out + z * batch_stride;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int m0 = mb + 32 * i + 8 * q + 4 * khalf;
                float ba[4] = {0.f, 0.f, 0.f, 0.f};
                if (bias) {
                    if (vec) {
                        const float4 b4 = *reinterpret_cast<const float4 *>(bias + m0);
                        ba[0] = b4.x, ba[1] = b4.y, ba[2] = b4.z, ba[3] = b4.w;
                    } else {
#pragma unroll
                        for (int p = 0; p < 4; ++p) ba[p] = bias[m0 + p];
                    }
                }
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    float *o = zo + (int64_t)m0 * N + nb + 32 * j + col;
#pragma unroll
                    for (int p = 0; p < 4; ++p) o[(int64_t)p * N] = act_apply(act, v[i][j][4 * q + p] + ba[p]);
                }
            }
    }
};

// GLU over channel pairs (c, C + c), plus the optional frequency embedding.
struct EpGlu : EpBase {
    float *out;
    const float *bias;
    const float *emb;  // (F, C) already scaled by emb_scale
    float emb_scale;
    int64_t batch_stride;
    int N, C, T;
    bool vec;  // bias 16-byte aligned and C a multiple of 4: glu_frags may read float4 biases
    __device__ void glu(int z, int c, int n, float v, float g) {
        float a = v + bias[c], gate = g + bias[C + c];
        float y = a * sigmoid(gate);
        if (emb) y += emb_scale * emb[(n / T) * C + c];
        out[z * batch_stride + (int64_t)c * N + n] = y;
    }
    // Whole fragments of a wave holding GCH value channels from cb and their
    // gates: the value rows of 8-row block b = 32 i + 8 q are channels
    // cb + b + 4 khalf + p (p = r % 4), their gates sit GCH rows further on
    // (fragment (b + GCH) / 32, register 4 ((b + GCH) % 32 / 8) + p). Each
    // block's four biases are one float4 (cb and C are multiples of 4; the
    // launcher checks C), and the embedding row is found once per column.
    static constexpr bool frags = true;
    template <int GCH, int TM, int TN>
    __device__ void glu_frags(int z, int cb, int nb, int col, int khalf, const floatx16 (&v)[TM][TN]) {
        if (!vec) {
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int b = 32 * i + 8 * (r / 4);
                        if (b >= GCH) continue;
                        const int gi = (b + GCH) / 32, gr = (((b + GCH) % 32) / 8) * 4 + r % 4;
                        glu(z, cb + b + 4 * khalf + r % 4, nb + 32 * j + col, v[i][j][r], v[gi][j][gr]);
                    }
            return;
        }
        float *zo = out + z * batch_stride;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int n = nb + 32 * j + col;
            const float *er = emb ? emb + (n / T) * C : nullptr;
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int b = 32 * i + 8 * q;
                    if (b >= GCH) continue;
                    const int gi = (b + GCH) / 32, gq = ((b + GCH) % 32) / 8;
                    const int c0 = cb + b + 4 * khalf;
                    const float4 bv = *reinterpret_cast<const float4 *>(bias + c0);
                    const float4 bg = *reinterpret_cast<const float4 *>(bias + C + c0);
                    const float bva[4] = {bv.x, bv.y, bv.z, bv.w}, bga[4] = {bg.x, bg.y, bg.z, bg.w};
#pragma unroll
                    for (int p = 0; p < 4; ++p) {
                        float y = (v[i][j][4 * q + p] + bva[p]) * sigmoid(v[gi][j][4 * gq + p] + bga[p]);
                        if (er) y += emb_scale * er[c0 + p];
                        zo[(int64_t)(c0 + p) * N + n] = y;
                    }
                }
        }
    }
};

// Transposed-conv output: row m = o * st + p, column n = qi * P + t is
// output position a = st * (q0 + qi) + p - crop of channel o (dropped
// outside the crop [0, a_out)).
struct EpConvT : EpBase {
    float *out;
    const float *bias;
    int oc, st, crop, a_out, P, q0, act;
    __device__ void store(int z, int m, int n, float v) {
        const int o = m / st, p = m - o * st;
        const int qi = n / P, t = n - qi * P;
        const int a = st * (q0 + qi) + p - crop;
        if (a < 0 || a >= a_out) return;
        out[(((int64_t)z * oc + o) * a_out + a) * P + t] = act_apply(act, v + bias[o]);
    }
    // Whole fragments (stride 4, the model's): register r of fragment (i, j)
    // is row mb + 32 i + 8 (r / 4) + 4 khalf + r % 4 with mb a multiple of 4,
    // i.e. channel mb / 4 + 8 i + 2 (r / 4) + khalf at phase r % 4, so the
    // column's (qi, t) and the four phases' output offsets are worked out
    // once per column instead of once per element.
    static constexpr bool frags = true;
    template <int TM, int TN>
    __device__ void store_frags(int z, int mb, int nb, int col, int khalf, const floatx16 (&v)[TM][TN]) {
        if (st != 4) {
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        store(z, mb + 32 * i + 8 * (r / 4) + 4 * khalf + r % 4, nb + 32 * j + col, v[i][j][r]);
            return;
        }
        const int64_t plane = (int64_t)a_out * P;
        float *zo = out + (int64_t)z * oc * plane;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int n = nb + 32 * j + col;
            const int qi = n / P, t = n - qi * P;
            const int a0 = 4 * (q0 + qi) - crop;
            int64_t off[4];
            bool ok[4];
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                ok[p] = a0 + p >= 0 && a0 + p < a_out;
                off[p] = (int64_t)(a0 + p) * P + t;
            }
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int o = mb / 4 + 8 * i + 2 * q + khalf;
                    const float bo = bias[o];
                    float *ro = zo + (int64_t)o * plane;
#pragma unroll
                    for (int p = 0; p < 4; ++p)
                        if (ok[p]) ro[off[p]] = act_apply(act, v[i][j][4 * q + p] + bo);
                }
        }
    }
};

// DConv conv1: y = conv + bias stored as (rows, H, T); GN statistics per row.
struct EpConv1 {
    float *y;
    const float *bias;
    double *stats;
    int H, T;
    MomentAcc acc;
    __device__ void init(int) {}
    __device__ void store(int z, int m, int n, float v) {
        float r = v + bias[m];
        y[((int64_t)z * H + m) * T + n] = r;
        acc.add(r);
    }
    __device__ void finalize(int z) { acc.flush(stats + 2 * z); }
};

// DConv conv2, first pass: GN statistics of (conv + bias), nothing stored.
struct EpConv2Stats {
    const float *bias;
    double *stats;
    bool vec;  // bias 16-byte aligned
    MomentAcc acc;
    __device__ void init(int) {}
    __device__ void store(int, int m, int, float v) { acc.add(v + bias[m]); }
    // Whole fragments: each run of four registers (four consecutive rows)
    // takes one float4 of biases and enters the f64 moments as one fp32
    // partial sum of four values and one of their squares.
    static constexpr bool frags = true;
    template <int TM, int TN>
    __device__ void store_frags(int, int mb, int, int, int khalf, const floatx16 (&v)[TM][TN]) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int m0 = mb + 32 * i + 8 * q + 4 * khalf;
                float ba[4];
                if (vec) {
                    const float4 b4 = *reinterpret_cast<const float4 *>(bias + m0);
                    ba[0] = b4.x, ba[1] = b4.y, ba[2] = b4.z, ba[3] = b4.w;
                } else {
#pragma unroll
                    for (int p = 0; p < 4; ++p) ba[p] = bias[m0 + p];
                }
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    float s4 = 0.0f, q4 = 0.0f;
#pragma unroll
                    for (int p = 0; p < 4; ++p) {
                        const float x = v[i][j][4 * q + p] + ba[p];
                        s4 += x;
                        q4 = fmaf(x, x, q4);
                    }
                    acc.s += (double)s4;
                    acc.q += (double)q4;
                }
            }
    }
    __device__ void finalize(int z) { acc.flush(stats + 2 * z); }
};

// DConv conv2's GroupNorm moments from the Gram matrix of its input (as the
// row kernel takes them), instead of a pass that computes conv2 for them:
// with y = W2 g + b2 over the row's T positions, S = sum_t g and G =
// sum_t g g^T,
//   sum y   = V . S + T sum(b2),                  V = sum_o w2[o]
//   sum y^2 = sum_mn P_mn G_mn + 2 U . S + T sum(b2^2),
//             P = W2^T W2, U = W2^T b2.
// `gram` holds P (H x H), U, V and (sum b2, sum b2^2) in f64 (dconv_gram_
// weights). The GEMM's rows 0..H-1 give G and row H (ones) gives S; each
// t-chunk of a row adds its share to the row's moments.
struct EpGramMoments {
    const double *gram;
    double *stats;
    int H, T, chunks;
    double s = 0.0, q = 0.0;
    __device__ void init(int) {}
    __device__ void store(int, int m, int n, float v) {
        const double *P = gram, *U = gram + H * H, *V = U + H;
        if (m < H) {
            q += P[m * H + n] * (double)v;
        } else {
            s += V[n] * (double)v;
            q += 2.0 * U[n] * (double)v;
        }
    }
    __device__ void finalize(int z) {
        const int row = z / chunks;
        if (z == row * chunks && threadIdx.x == 0) {
            const double *c = gram + H * H + 2 * H;
            s += (double)T * c[0];
            q += (double)T * c[1];
        }
        block_moments_atomic(s, q, stats + 2 * row);
    }
};

// DConv conv2, second pass: GN -> GLU -> LayerScale -> residual add into x,
// whose rows (b, f) live in a (B, C, F, T) tensor.
// Per-channel affines of the conv2 epilogue, one table per workgroup.
constexpr int C2A_MAXC = 768;
__shared__ float4 c2a_affine[C2A_MAXC];

struct EpConv2Apply {
    float *x;
    const float *bias, *nw, *nb, *gamma;
    const double *stats;
    int C, F, T;
    float *xz;  // this row's (b, f) plane origin in x
    // GN2 of the row and the channel's bias, GN affine and LayerScale fold
    // into value' = v * a.x + a.y (LayerScale included) and gate' = g * a.z + a.w,
    // one float4 per channel in LDS: the element loop then reads one LDS
    // quad per element instead of seven scattered parameters. (The kernel's
    // first barrier comes before its epilogue.)
    __device__ void init(int z) {
        float mean, inv;
        gn_stats(stats + 2 * z, 2.0 * C * (double)T, mean, inv);
        for (int c = threadIdx.x; c < C; c += blockDim.x) {
            const float vs = inv * nw[c], gs = inv * nw[C + c];
            const float vsh = (bias[c] - mean) * vs + nb[c], gsh = (bias[C + c] - mean) * gs + nb[C + c];
            c2a_affine[c] = make_float4(gamma[c] * vs, gamma[c] * vsh, gs, gsh);
        }
        const int b = z / F, f = z - b * F;
        xz = x + ((int64_t)b * C * F + f) * T;
    }
    __device__ void glu(int, int c, int n, float v, float g) {
        const float4 a = c2a_affine[c];
        float *dst = xz + (int64_t)c * F * T + n;
        *dst += fmaf(v, a.x, a.y) * sigmoid(fmaf(g, a.z, a.w));
    }
    __device__ void finalize(int) {}
};

// Linear tails on token rows. With `planes` set (bias or bias + GELU tails
// only) the results are written as that many bf16 planes, plane_stride
// apart, for a following linear that reads planes; `out` is then unused.
struct EpLinear {
    float *out;
    const float *bias, *residual, *gamma;
    double *stats;
    int64_t ldo, batch_stride;
    int tail;
    MomentAcc acc;
    __device__ void init(int) {}
    __device__ void store(int z, int m, int n, float v) {
        int64_t at = z * batch_stride + (int64_t)m * ldo + n;
        float a = v + bias[n];
        if (tail == TAIL_BIAS_GELU) {
            a = gelu(a);
        } else if (tail == TAIL_RESIDUAL_SCALE) {
            a = residual[at] + a * gamma[n];
            if (stats) acc.add(a);
        }
        out[at] = a;
    }
    // A wave's TM x TN fragments of a tile that lies wholly in range:
    // fragment (i, j) register r is row mb + 32 i + 8 (r / 4) + 4 khalf + r % 4,
    // column nb + 32 j + col. The residual rows are all loaded before the
    // first is used, so the loads overlap instead of each waiting in turn.
    template <int TM, int TN>
    __device__ void store_frags(int z, int mb, int nb, int col, int khalf, const floatx16 (&v)[TM][TN]) {
        float *o = out + z * batch_stride;
        const float *res = residual ? residual + z * batch_stride : nullptr;
        auto at = [&](int i, int j, int r) -> int64_t {
            return (int64_t)(mb + 32 * i + 8 * (r / 4) + 4 * khalf + r % 4) * ldo + nb + 32 * j + col;
        };
        if (tail == TAIL_RESIDUAL_SCALE) {
            // One fragment row (TN x 16 residuals) in flight at a time keeps
            // the register count at the main loop's.
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                float rv[TN][16];
#pragma unroll
                for (int j = 0; j < TN; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r) rv[j][r] = res[at(i, j, r)];
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    const float bn = bias[nb + 32 * j + col], gn = gamma[nb + 32 * j + col];
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const float a = rv[j][r] + (v[i][j][r] + bn) * gn;
                        if (stats) acc.add(a);
                        o[at(i, j, r)] = a;
                    }
                }
            }
        } else if (tail == TAIL_BIAS_GELU) {
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const float bn = bias[nb + 32 * j + col];
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int r = 0; r < 16; ++r) o[at(i, j, r)] = gelu(v[i][j][r] + bn);
            }
        } else {
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const float bn = bias[nb + 32 * j + col];
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int r = 0; r < 16; ++r) o[at(i, j, r)] = v[i][j][r] + bn;
            }
        }
    }
    __device__ void finalize(int z) {
        if (stats) acc.flush(stats + 2 * z);
    }
};

// Epilogue of a linear whose output feeds the next plane GEMM (the
// transformer FFN's first linear): GELU(acc + bias) as P bf16 planes, plane
// q at out + q * plane_stride. A fixed tail and plane count keep the stores
// branch-free, so the GELU chains of neighbouring elements interleave;
// registers r and r + 1 (rows m and m + 1 of one column) share one
// v_cvt_pk_bf16_f32 per plane.
template <int P>
struct EpGeluPlanes {
    unsigned short *out;
    const float *bias;
    int64_t ldo, batch_stride, plane_stride;
    __device__ void init(int) {}
    __device__ void finalize(int) {}
    __device__ void store(int z, int m, int n, float v) {
        store_planes1<P>(out + z * batch_stride + (int64_t)m * ldo + n, plane_stride, gelu(v + bias[n]));
    }
    // Each plane's base is the wave tile's first row, and a lane's offsets
    // within the tile are 32-bit (the host keeps 256 rows of ldo below 2^31),
    // so no 64-bit address per store stays live.
    template <int TM, int TN>
    __device__ __forceinline__ void store_frags(int z, int mb, int nb, int col, int khalf,
                                                const floatx16 (&v)[TM][TN]) {
        unsigned short *base[P];
#pragma unroll
        for (int q = 0; q < P; ++q) base[q] = out + q * plane_stride + z * batch_stride + (int64_t)mb * ldo + nb;
        const unsigned ld = (unsigned)ldo, lane = 4 * khalf * ld + col;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const float bn = bias[nb + 32 * j + col];
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int r = 0; r < 16; r += 2) {
                    const unsigned off = lane + (32 * i + 8 * (r / 4) + r % 4) * ld + 32 * j;
                    unsigned w[P];
                    split_pair_planes<P>(gelu(v[i][j][r] + bn), gelu(v[i][j][r + 1] + bn), w);
#pragma unroll
                    for (int q = 0; q < P; ++q) {
                        base[q][off] = (unsigned short)w[q];
                        base[q][off + ld] = (unsigned short)(w[q] >> 16);
                    }
                    // Four elements in flight at a time.
                    if (r % 4 == 2) __builtin_amdgcn_sched_barrier(0);
                }
        }
    }
};

// ---------------------------------------------------------------------------
// Tile selection
// ---------------------------------------------------------------------------

// Direct-to-LDS linear kernel: k-tiles in flight (0 = use gemm_kernel), block
// tile and waves along M.
#ifndef DMX_DMA_STAGES
#define DMX_DMA_STAGES 4
#endif
#ifndef DMX_DMA_BM
#define DMX_DMA_BM 128
#endif
#ifndef DMX_DMA_BN
#define DMX_DMA_BN 128
#endif
#ifndef DMX_DMA_WM
#define DMX_DMA_WM 2
#endif

// Column tile of the 48-channel GLU shapes.
#ifndef DMX_GLU96_BN
#define DMX_GLU96_BN 64
#endif
#ifndef DMX_GLU48_BN
#define DMX_GLU48_BN 128
#endif

// PREC (gemm_kernel's): the three-plane mode serves the tiles it measured
// faster on (the 192- and 96-row tiles of the encoder convs, the GLU
// rewrites and the transposed convs: 8-20 % per kernel on MI355X); the
// narrow tiles (32 and 64 rows, whose MFMA work per loaded element is
// small) and the DConv conv2 loader (GroupNorm + GELU on load, VALU-bound)
// measured 5-70 % slower with it and stay on the fp32 matrix cores.
template <bool GLU, int PREC, class AL, class BL, class EP>
void gemm_pick(hipStream_t s, int M, int N, int K, int batches, const AL &al, const BL &bl, const EP &ep) {
    constexpr int BIG = (PREC == 3 && std::is_same<BL, NormGeluQuads>::value) ? 0 : PREC;
    constexpr int NARROW = PREC == 3 ? 0 : PREC;
    if constexpr (GLU) {
        // M = C output channels; a block covers BM / 2 of them.
        if (M % 96 == 0)
            launch_gemm<192, DMX_GLU96_BN, 2, true, BIG>(s, M, N, K, batches, al, bl, ep);  // 2 x 48 channels
        else if (M == 48)
            launch_gemm<96, DMX_GLU48_BN, 1, true, BIG>(s, M, N, K, batches, al, bl, ep);   // 1 x 48 channels
        else if (M > 32)
            launch_gemm<128, 128, 2, true, BIG>(s, M, N, K, batches, al, bl, ep);  // 2 x 32 channels
        else
            launch_gemm<64, 128, 1, true, NARROW>(s, M, N, K, batches, al, bl, ep);
    } else {
#ifdef DMX_BIG_BM  // tuning builds only: a larger tile for tall problems
        if (M >= DMX_BIG_BM)
            launch_gemm<DMX_BIG_BM, DMX_BIG_BN, DMX_BIG_WM, false, BIG>(s, M, N, K, batches, al, bl, ep);
        else
#endif
        if (M % 96 == 0 && M >= 192 && M <= 768)  // channel counts 192, 384, 768: 96-row wave tiles
            launch_gemm<192, 64, 2, false, BIG>(s, M, N, K, batches, al, bl, ep);
        else if (M == 96)
            launch_gemm<96, 128, 1, false, BIG>(s, M, N, K, batches, al, bl, ep);
        else if (M >= 96)
            launch_gemm<128, 128, 2, false, BIG>(s, M, N, K, batches, al, bl, ep);
        else if (M > 32) {
            // 64-row tiles: 64-wide columns when 128-wide ones would leave CUs idle.
            if (ceil_div(N, 128) * ceil_div(M, 64) * batches < 256)
                launch_gemm<64, 64, 2, false, NARROW>(s, M, N, K, batches, al, bl, ep);
            else
                launch_gemm<64, 128, 2, false, NARROW>(s, M, N, K, batches, al, bl, ep);
        } else {
            // 32-row tiles: 128-wide columns unless 256-wide ones fill two rounds
            // of the CUs with little padding (short rows such as T = 336 pad a
            // 256-wide tile by a third).
            const int64_t n256 = ceil_div(N, 256) * 256;
            if (ceil_div(N, 256) * batches >= 512 && 5 * n256 <= 6 * (int64_t)N)
                launch_gemm<32, 256, 1, false, NARROW>(s, M, N, K, batches, al, bl, ep);
            else
                launch_gemm<32, 128, 1, false, NARROW>(s, M, N, K, batches, al, bl, ep);
        }
    }
}

// The fp32 precision's convolutions run on three bf16 planes per operand
// unless DMX_CONV_PLANES=0 (read once) keeps them on the fp32 matrix cores.
bool conv_planes_enabled() {
    static const bool on = [] {
        const char *e = std::getenv("DMX_CONV_PLANES");
        return !e || std::atoi(e) != 0;
    }();
    return on;
}

// Contractions take bf16 MFMA inputs, or three bf16 planes, when the calling
// thread's precision scope says so (fp32 accumulation and epilogues either
// way).
template <bool GLU, class AL, class BL, class EP>
void gemm_auto(hipStream_t s, int M, int N, int K, int batches, const AL &al, const BL &bl, const EP &ep) {
    if (bf16_mfma())
        gemm_pick<GLU, 1>(s, M, N, K, batches, al, bl, ep);
    else if (mfma_precision() == MfmaPrecision::FP32X3 && conv_planes_enabled())
        gemm_pick<GLU, 3>(s, M, N, K, batches, al, bl, ep);
    else
        gemm_pick<GLU, 0>(s, M, N, K, batches, al, bl, ep);
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

KMajor kmajor(const float *p, int64_t ld, int64_t batch_stride) {
    return KMajor{p, ld, batch_stride, aligned16(p) && ld % 4 == 0 && batch_stride % 4 == 0};
}

template <int KH, int KW>
ConvGather<KH, KW> gather(const float *x, const float *skip, int64_t outer, int64_t inner, int zdiv, int ic_stride_h,
                          int h, int w, int kh, int kw, int sh, int sw, int ph, int pw, int dh, int dw, int ow) {
    ConvGather<KH, KW> g;
    g.x = x;
    g.skip = skip;
    g.outer = outer;
    g.inner = inner;
    g.cs = (int64_t)ic_stride_h * w;
    g.zdiv = zdiv;
    g.h = h;
    g.w = w;
    g.kh_rt = kh;
    g.kw_rt = kw;
    g.sh = sh;
    g.sw = sw;
    g.ph = ph;
    g.pw = pw;
    g.dh = dh;
    g.dw = dw;
    g.ow = ow;
    return g;
}

template <int KH, int KW, bool SKIP>
ConvGatherTM<KH, KW, SKIP> gather_tm(const float *x, const float *skip, int64_t outer, int64_t inner, int zdiv,
                                     int ic_stride_h, int h, int w, int sh, int sw, int ph, int pw, int dh, int dw,
                                     int ow, int kh, int kw) {
    ConvGatherTM<KH, KW, SKIP> g;
    g.kh_rt = kh;
    g.kw_rt = kw;
    g.x = x;
    g.skip = skip;
    g.outer = outer;
    g.inner = inner;
    g.cs = (int64_t)ic_stride_h * w;
    g.zdiv = zdiv;
    g.h = h;
    g.w = w;
    g.sh = sh;
    g.sw = sw;
    g.ph = ph;
    g.pw = pw;
    g.dh = dh;
    g.dw = dw;
    g.ow = ow;
    return g;
}

// Runs a conv GEMM with a compile-time kernel when it is one of the model's.
// K = ic * kh * kw; the weight rows are in GEMM order (tap-major when
// conv_tap_major(ic, kh, kw)).
template <bool GLU, class EP>
void conv_dispatch(hipStream_t s, int M, int N, int K, int batches, const KMajor &wa, const float *x,
                   const float *skip, int64_t outer, int64_t inner, int zdiv, int ic_stride_h, int h, int w, int kh,
                   int kw, int sh, int sw, int ph, int pw, int dh, int dw, int ow, const EP &ep) {
    require_ptrs({x, wa.p}, "conv");
    const int ic = K / (kh * kw);
    DMX_REQUIRE(ic * kh * kw == K, "conv: K is not ic * kh * kw");
    if (conv_tap_major(ic, kh, kw)) {
#define DMX_CONV_TM_CASE(A, B, S)                                                                          \
    if (kh == A && kw == B && (skip != nullptr) == S) {                                                      \
        gemm_auto<GLU>(s, M, N, K, batches, wa,                                                              \
                       gather_tm<A, B, S>(x, skip, outer, inner, zdiv, ic_stride_h, h, w, sh, sw, ph, pw, dh,  \
                                          dw, ow, kh, kw),                                                   \
                       ep);                                                                                  \
        return;                                                                                              \
    }
        // Encoders and DConv gather without a skip; decoder rewrites with one.
        DMX_CONV_TM_CASE(8, 1, false)
        DMX_CONV_TM_CASE(1, 8, false)
        DMX_CONV_TM_CASE(3, 3, true)
        DMX_CONV_TM_CASE(1, 3, true)
        DMX_CONV_TM_CASE(1, 3, false)
#undef DMX_CONV_TM_CASE
        if (skip)
            gemm_auto<GLU>(s, M, N, K, batches, wa,
                           gather_tm<0, 0, true>(x, skip, outer, inner, zdiv, ic_stride_h, h, w, sh, sw, ph, pw, dh,
                                                 dw, ow, kh, kw),
                           ep);
        else
            gemm_auto<GLU>(s, M, N, K, batches, wa,
                           gather_tm<0, 0, false>(x, skip, outer, inner, zdiv, ic_stride_h, h, w, sh, sw, ph, pw, dh,
                                                  dw, ow, kh, kw),
                           ep);
        return;
    }
    // A pointwise conv without skip is a plain GEMM over (ic, positions).
    if (kh == 1 && kw == 1 && sh == 1 && sw == 1 && ph == 0 && pw == 0 && !skip && zdiv == 1 && ow == w) {
        gemm_auto<GLU>(s, M, N, K, batches, wa, MNMajor{x, (int64_t)ic_stride_h * w, outer}, ep);
        return;
    }
#define DMX_CONV_CASE(A, B)                                                                                \
    if (kh == A && kw == B) {                                                                                \
        gemm_auto<GLU>(s, M, N, K, batches, wa,                                                              \
                       gather<A, B>(x, skip, outer, inner, zdiv, ic_stride_h, h, w, kh, kw, sh, sw, ph, pw, dh, \
                                    dw, ow),                                                                 \
                       ep);                                                                                  \
        return;                                                                                              \
    }
    DMX_CONV_CASE(8, 1)
    DMX_CONV_CASE(1, 8)
    DMX_CONV_CASE(3, 3)
    DMX_CONV_CASE(1, 3)
    DMX_CONV_CASE(1, 1)
#undef DMX_CONV_CASE
    gemm_auto<GLU>(s, M, N, K, batches, wa,
                   gather<0, 0>(x, skip, outer, inner, zdiv, ic_stride_h, h, w, kh, kw, sh, sw, ph, pw, dh, dw, ow), ep);
}

}  // namespace

// ---------------------------------------------------------------------------
// Launchers
// ---------------------------------------------------------------------------

void conv2d(hipStream_t s, const float *x, const float *skip, int b, int ic, int h, int w, const float *weight,
            const float *bias, int oc, int kh, int kw, int sh, int sw, int ph, int pw, int dh, int dw, float *out,
            Act act) {
    int eh = dh * (kh - 1) + 1, ew = dw * (kw - 1) + 1;
    DMX_REQUIRE(h + 2 * ph >= eh && w + 2 * pw >= ew, "conv2d: kernel larger than the padded input");
    int oh = (h + 2 * ph - eh) / sh + 1, ow = (w + 2 * pw - ew) / sw + 1;
    int K = ic * kh * kw, N = oh * ow;
    EpChannels ep;
    ep.out = out;
    ep.bias = bias;
    ep.batch_stride = (int64_t)oc * N;
    ep.N = N;
    ep.act = act;
    ep.vec = !ep.bias || aligned16(ep.bias);
    conv_dispatch<false>(s, oc, N, K, b, kmajor(weight, K, 0), x, skip, (int64_t)ic * h * w, 0, 1, h, h, w, kh, kw, sh,
                         sw, ph, pw, dh, dw, ow, ep);
}

void conv1d_right_padded(hipStream_t s, const float *x, int b, int ic, int len, int len_padded, const float *weight,
                         const float *bias, int oc, int k, int stride, int pad, float *out, Act act) {
    DMX_REQUIRE(len_padded >= len && len_padded + 2 * pad >= k, "conv1d_right_padded: bad lengths");
    int ow = (len_padded + 2 * pad - k) / stride + 1;
    int K = ic * k;
    EpChannels ep;
    ep.out = out;
    ep.bias = bias;
    ep.batch_stride = (int64_t)oc * ow;
    ep.N = ow;
    ep.act = act;
    ep.vec = !ep.bias || aligned16(ep.bias);
    // Bounds use the unpadded length: the right pad is zeros either way.
    conv_dispatch<false>(s, oc, ow, K, b, kmajor(weight, K, 0), x, nullptr, (int64_t)ic * len, 0, 1, 1, 1, len, 1, k, 1,
                         stride, 0, pad, 1, 1, ow, ep);
}

void conv2d_glu(hipStream_t s, const float *x, const float *skip, int b, int ic, int h, int w, const float *weight,
                const float *bias, int C, int kh, int kw, int ph, int pw, float *out, const float *emb,
                float emb_scale) {
    require_ptrs({bias, out}, "conv2d_glu");
    int oh = h + 2 * ph - kh + 1, ow = w + 2 * pw - kw + 1;
    DMX_REQUIRE(oh > 0 && ow > 0, "conv2d_glu: kernel larger than the padded input");
    int K = ic * kh * kw, N = oh * ow;
    EpGlu ep;
    ep.out = out;
    ep.bias = bias;
    ep.emb = emb;
    ep.emb_scale = emb_scale;
    ep.batch_stride = (int64_t)C * N;
    ep.N = N;
    ep.C = C;
    ep.T = ow;
    ep.vec = aligned16(bias) && C % 4 == 0;
    conv_dispatch<true>(s, C, N, K, b, kmajor(weight, K, 0), x, skip, (int64_t)ic * h * w, 0, 1, h, h, w, kh, kw, 1, 1,
                        ph, pw, 1, 1, ow, ep);
}

void conv_gemm_weights(const float *w, int oc, int ic, int kh, int kw, float *out) {
    const int taps = kh * kw;
    const bool tm = conv_tap_major(ic, kh, kw);
    for (int o = 0; o < oc; ++o)
        for (int c = 0; c < ic; ++c)
            for (int t = 0; t < taps; ++t) {
                const int64_t src = ((int64_t)o * ic + c) * taps + t;
                const int64_t dst = tm ? (int64_t)o * ic * taps + ((int64_t)(c / 4) * taps + t) * 4 + c % 4 : src;
                out[dst] = w[src];
            }
}

int conv_transpose_taps(int k, int st) { return (k + st - 1) / st; }

void pack_conv_transpose(const float *w, int ic, int oc, int k, int st, float *packed) {
    int taps = conv_transpose_taps(k, st);
    for (int p = 0; p < st; ++p)
        for (int o = 0; o < oc; ++o)
            for (int c = 0; c < ic; ++c)
                for (int j = 0; j < taps; ++j) {
                    int kk = p + st * j;
                    packed[((int64_t)(p * oc + o) * ic + c) * taps + j] = kk < k ? w[((int64_t)c * oc + o) * k + kk] : 0.0f;
                }
}

void conv_transpose_axis(hipStream_t s, const float *x, int b, int ic, int A, int P, const float *weight_packed,
                         const float *bias, int oc, int k, int st, int crop, int a_out, float *out, Act act) {
    require_ptrs({x, weight_packed, bias, out}, "conv_transpose_axis");
    int taps = conv_transpose_taps(k, st);
    DMX_REQUIRE(taps == 2 && k == 2 * st, "conv_transpose_axis: only kernel = 2 * stride is supported");
    DMX_REQUIRE(crop >= 0 && crop + a_out <= (A - 1) * st + k, "conv_transpose_axis: crop past the produced length");
    DMX_REQUIRE(ic % 2 == 0, "conv_transpose_axis: the input channel count must be even (k quads are 2 channels)");
    // Input rows q cover every kept output a = st * q + p - crop, p < st.
    const int q0 = crop >= st - 1 ? (crop - (st - 1) + st - 1) / st : 0;
    const int q_end = (a_out + crop + st - 1) / st;
    const int K = ic * taps, N = (q_end - q0) * P, M = oc * st;
    ConvTGather g{x, ic, A, P, q0};
    PhaseWeights pw{weight_packed, st, oc, K, aligned16(weight_packed) && K % 4 == 0};
    EpConvT ep;
    ep.out = out;
    ep.bias = bias;
    ep.oc = oc;
    ep.st = st;
    ep.crop = crop;
    ep.a_out = a_out;
    ep.P = P;
    ep.q0 = q0;
    ep.act = act;
    gemm_auto<false>(s, M, N, K, b, pw, g, ep);
}

// P = W2^T W2 (H x H), U = W2^T b2, V = sum_o W2[o], then (sum b2,
// sum b2^2), in f64, for conv2's moments from a Gram matrix (EpGramMoments);
// w2 is (O, H). One thread per output.
__global__ void dconv_gram_weights_kernel(const float *__restrict__ w2, const float *__restrict__ b2, int O, int H,
                                          double *__restrict__ out) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    const int n = H * H + 2 * H + 2;
    if (i >= n) return;
    double acc = 0.0;
    if (i < H * H) {
        const int m = i / H, k = i - m * H;
        for (int o = 0; o < O; ++o) acc += (double)w2[(int64_t)o * H + m] * (double)w2[(int64_t)o * H + k];
    } else if (i < H * H + H) {
        const int m = i - H * H;
        for (int o = 0; o < O; ++o) acc += (double)w2[(int64_t)o * H + m] * (double)b2[o];
    } else if (i < H * H + 2 * H) {
        const int m = i - H * H - H;
        for (int o = 0; o < O; ++o) acc += (double)w2[(int64_t)o * H + m];
    } else {
        const bool squares = i == n - 1;
        for (int o = 0; o < O; ++o) acc += squares ? (double)b2[o] * (double)b2[o] : (double)b2[o];
    }
    out[i] = acc;
}

int64_t dconv_gram_doubles(int H) { return (int64_t)H * H + 2 * H + 2; }

void dconv_gram_weights(hipStream_t s, const float *w2, const float *b2, int C, int H, double *out) {
    require_ptrs({w2, b2, out}, "dconv_gram_weights");
    const int n = (int)dconv_gram_doubles(H);
    hipLaunchKernelGGL(dconv_gram_weights_kernel, dim3((unsigned)ceil_div(n, 256)), dim3(256), 0, s, w2, b2, 2 * C, H,
                       out);
    DMX_LAUNCH_CHECK();
}

// Positions per t-chunk of the Gram launch: 8 k-tiles of MFMA work per block.
constexpr int GRAM_CHUNK = 128;

void dconv_layer(hipStream_t s, float *x, int B, int C, int F, int T, int dil, const float *w1,
                 const float *w1_gemm, const float *w1_t, const float *b1, int H, const float *n1w,
                 const float *n1b, const float *w2, const float *b2, const float *n2w, const float *n2b,
                 const float *gamma, const double *gram, float *hbuf, double *stats) {
    require_ptrs({x, w1, w1_gemm, b1, n1w, n1b, w2, b2, n2w, n2b, gamma, hbuf, stats}, "dconv_layer");
    const int rows = B * F;
    DMX_REQUIRE(rows <= 65535, "dconv_layer: too many rows for one launch");
    DMX_REQUIRE(C <= C2A_MAXC, "dconv_layer: more channels than the conv2 epilogue's table holds");
    if (dconv_narrow_applies(C, H)) {
        dconv_layer_narrow(s, x, B, C, F, T, dil, w1, w1_t, b1, H, n1w, n1b, w2, b2, n2w, n2b, gamma, hbuf);
        return;
    }
    double *st1 = stats, *st2 = stats + 2 * rows;
    zero_doubles(s, stats, 4 * (int64_t)rows);
    // conv1: k3, dilation dil, padding dil, over t; rows (b, f) as the batch.
    EpConv1 e1;
    e1.y = hbuf;
    e1.bias = b1;
    e1.stats = st1;
    e1.H = H;
    e1.T = T;
    conv_dispatch<false>(s, H, T, C * 3, rows, kmajor(w1_gemm, C * 3, 0), x, nullptr, (int64_t)C * F * T, T, F, F, 1, T,
                         1, 3, 1, 1, 0, dil, 1, dil, T, e1);
    // conv2's GroupNorm moments: from the Gram matrix of its input when the
    // folded weights are given, else from a pass that computes conv2 for them.
    EpConv2Stats e2;
    e2.bias = b2;
    e2.stats = st2;
    e2.vec = aligned16(b2);
    const bool by_gram = gram != nullptr && H + 1 <= 64;
    if (by_gram) {
        const int chunks = (int)ceil_div(T, GRAM_CHUNK);
        DMX_REQUIRE((int64_t)rows * chunks <= 65535, "dconv_layer: too many Gram blocks");
        EpGramMoments eg;
        eg.gram = gram;
        eg.stats = st2;
        eg.H = H;
        eg.T = T;
        eg.chunks = chunks;
        GramRows g{hbuf, st1, n1w, n1b, H, T, GRAM_CHUNK, chunks};
        launch_gemm<64, 64, 2, false, false>(s, H + 1, H, GRAM_CHUNK, rows * chunks, g, g, eg);
    }
    // Then GN + GLU + LayerScale + residual.
    EpConv2Apply e3;
    e3.x = x;
    e3.bias = b2;
    e3.nw = n2w;
    e3.nb = n2b;
    e3.gamma = gamma;
    e3.stats = st2;
    e3.C = C;
    e3.F = F;
    e3.T = T;
    if (H % 4 == 0) {
        NormGeluQuads ng{hbuf, st1, n1w, n1b, H, T};
        if (!by_gram) gemm_auto<false>(s, 2 * C, T, H, rows, kmajor(w2, H, 0), ng, e2);
        gemm_auto<true>(s, C, T, H, rows, kmajor(w2, H, 0), ng, e3);
    } else {
        NormGeluRows ng{hbuf, st1, n1w, n1b, H, T};
        if (!by_gram) gemm_auto<false>(s, 2 * C, T, H, rows, kmajor(w2, H, 0), ng, e2);
        gemm_auto<true>(s, C, T, H, rows, kmajor(w2, H, 0), ng, e3);
    }
}

void pointwise(hipStream_t s, const float *w, const float *bias, const float *x, int batches, int M, int K, int N,
               float *out, Act act) {
    require_ptrs({w, x, out}, "pointwise");
    EpChannels ep;
    ep.out = out;
    ep.bias = bias;
    ep.batch_stride = (int64_t)M * N;
    ep.N = N;
    ep.act = act;
    ep.vec = !ep.bias || aligned16(ep.bias);
    gemm_auto<false>(s, M, N, K, batches, kmajor(w, K, 0), MNMajor{x, N, (int64_t)K * N}, ep);
}

void linear(hipStream_t s, const float *x, int64_t ldx, int64_t x_batch_stride, const float *w, const float *bias,
            int batches, int M, int K, int N, float *out, int64_t ldo, int64_t out_batch_stride, LinearTail tail,
            const float *residual, const float *gamma, double *stats) {
    require_ptrs({x, w, bias, out}, "linear");
    if (tail == TAIL_RESIDUAL_SCALE) require_ptrs({residual, gamma}, "linear residual");
    EpLinear ep;
    ep.out = out;
    ep.bias = bias;
    ep.residual = residual;
    ep.gamma = gamma;
    ep.stats = stats;
    ep.ldo = ldo;
    ep.batch_stride = out_batch_stride;
    ep.tail = tail;
    const bool dma_ok = !bf16_mfma() && K % 16 == 0 && aligned16(x) && aligned16(w) &&
                        ldx % 4 == 0 && x_batch_stride % 4 == 0;
#if DMX_DMA_STAGES > 0
    if (dma_ok) {
        launch_gemm_dma<DMX_DMA_BM, DMX_DMA_BN, DMX_DMA_WM, DMX_DMA_STAGES>(
            s, M, N, K, batches, KMajorRows{x, ldx, x_batch_stride}, KMajorRows{w, K, 0}, ep);
        return;
    }
#else
    (void)dma_ok;
#endif
    gemm_auto<false>(s, M, N, K, batches, kmajor(x, ldx, x_batch_stride), kmajor(w, K, 0), ep);
}

// The in-projection's tail for the three-plane attention: column n of row m
// (token m of batch z) plus bias goes to q (fp32 rows of D) for n < q_cols,
// to the K planes for the next D columns and to the V^T planes for the last
// D (KVPlanes layout). Fragment columns lie in one of the three ranges, D
// being a multiple of 32; four consecutive fragment rows are four tokens
// that stay adjacent in the V^T token order.
struct EpQKV {
    float *q;
    int64_t q_bs;
    const float *bias;
    KVPlanes kv;
    int q_cols, D;
    __device__ void init(int) {}
    __device__ void finalize(int) {}
    __device__ void store(int z, int m, int n, float v) {
        const float a = v + bias[n];
        if (n < q_cols) {
            q[z * q_bs + (int64_t)m * D + n] = a;
        } else if (n < q_cols + D) {
            store_planes1<3>(kv.k + z * kv.k_bs + (int64_t)m * kv.ldk + (n - q_cols), kv.k_stride, a);
        } else {
            const int c = n - q_cols - D;
            store_planes1<3>(kv.vt + ((int64_t)z * D + c) * kv.ldvt + vt_token_pos(m), kv.vt_stride, a);
        }
    }
    template <int TM, int TN>
    __device__ void store_frags(int z, int mb, int nb, int col, int khalf, const floatx16 (&v)[TM][TN]) {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int n = nb + 32 * j + col;
            const float bn = bias[n];
            if (n < q_cols) {
                float *o = q + z * q_bs + n;
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        o[(int64_t)(mb + 32 * i + 8 * (r / 4) + 4 * khalf + r % 4) * D] = v[i][j][r] + bn;
            } else if (n < q_cols + D) {
                unsigned short *o = kv.k + z * kv.k_bs + (n - q_cols);
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        store_planes1<3>(o + (int64_t)(mb + 32 * i + 8 * (r / 4) + 4 * khalf + r % 4) * kv.ldk,
                                         kv.k_stride, v[i][j][r] + bn);
            } else {
                unsigned short *o = kv.vt + ((int64_t)z * D + (n - q_cols - D)) * kv.ldvt;
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int a4 = 0; a4 < 4; ++a4) {
                        const int t0 = mb + 32 * i + 8 * a4 + 4 * khalf;
                        store_planes4<3>(o + vt_token_pos(t0), kv.vt_stride,
                                         make_float4(v[i][j][4 * a4] + bn, v[i][j][4 * a4 + 1] + bn,
                                                     v[i][j][4 * a4 + 2] + bn, v[i][j][4 * a4 + 3] + bn));
                    }
            }
        }
    }
};

// Tiles of the plane GEMM (MI355X sweeps of the model's shapes). Three
// planes, 64-byte k-tiles, two stages:
// - N >= 2048: 256 x 128 on eight waves, N >= 1024: 128 x 256 on eight waves
//   (144 KB of LDS, one block and two waves per SIMD per CU);
// - N < 1024: 128 x 128 on eight waves when that grid fills two rounds of
//   the 256 CUs, else 256 x 128 for long contractions and 128 x 64 on four
//   waves for short ones.
// One plane: 128 x 128 (128 x 64 for small grids) on four waves with
// four-k-group tiles.
template <class EP>
void launch_linear_planes(hipStream_t s, int M, int N, int K, int batches, const PlaneRows &al, const PlaneRows &bl,
                          int P, const EP &ep) {
    const int64_t tiles = ceil_div((int64_t)M, (int64_t)128) * ceil_div((int64_t)N, (int64_t)128) * batches;
    if (P == 3) {
        DMX_REQUIRE(K % 32 == 0, "linear_planes: K must be a multiple of 32");
        if (N >= 2048)
            launch_gemm_planes<256, 128, 4, 2, 3, 32, 8>(s, M, N, K, batches, al, bl, ep);
        else if (N >= 1024)
            launch_gemm_planes<128, 256, 2, 2, 3, 32, 8>(s, M, N, K, batches, al, bl, ep);
        else if (tiles >= 512)
            launch_gemm_planes<128, 128, 4, 2, 3, 32, 8>(s, M, N, K, batches, al, bl, ep);
        else if (K >= 2048)
            launch_gemm_planes<256, 128, 4, 2, 3, 32, 8>(s, M, N, K, batches, al, bl, ep);
        else
            launch_gemm_planes<128, 64, 2, 2, 3, 32, 4>(s, M, N, K, batches, al, bl, ep);
    } else {
        DMX_REQUIRE(K % 64 == 0, "linear_planes: K must be a multiple of 64");
        if (tiles < 512 && N % 64 == 0)
            launch_gemm_planes<128, 64, 2, 3, 1, 64, 4>(s, M, N, K, batches, al, bl, ep);
        else
            launch_gemm_planes<128, 128, 2, 2, 1, 64, 4>(s, M, N, K, batches, al, bl, ep);
    }
}

void linear_planes(hipStream_t s, Planes x, int64_t ldx, int64_t x_batch_stride, Planes w, const float *bias,
                   int batches, int M, int K, int N, float *out, Planes out_planes, int64_t ldo,
                   int64_t out_batch_stride, LinearTail tail, const float *residual, const float *gamma,
                   double *stats) {
    require_ptrs({x.p, w.p, bias}, "linear_planes");
    DMX_REQUIRE(x.count == w.count && (x.count == 1 || x.count == 3), "linear_planes: 1 or 3 planes on both operands");
    if (out_planes.p) {
        DMX_REQUIRE(tail == TAIL_BIAS_GELU && out_planes.count == x.count,
                    "linear_planes: plane outputs take the bias + GELU tail and the operands' plane count");
        DMX_REQUIRE(out_planes.count == 1 || out_planes.stride >= (int64_t)batches * out_batch_stride,
                    "linear_planes: output planes overlap");
        DMX_REQUIRE(ldo > 0 && ldo * 256 < (1LL << 31), "linear_planes: plane output rows too long");
    } else {
        require_ptrs({out}, "linear_planes");
    }
    if (tail == TAIL_RESIDUAL_SCALE) require_ptrs({residual, gamma}, "linear residual");
    // Batches laid end to end are one taller problem (whole tiles run over
    // the batch boundaries), unless the epilogue keeps per-batch moments.
    int64_t obs = out_batch_stride;
    if (batches > 1 && !stats && x_batch_stride == (int64_t)M * ldx && out_batch_stride == (int64_t)M * ldo &&
        (int64_t)M * batches < (1LL << 31)) {
        M *= batches;
        batches = 1;
        obs = 0;
    }
    const PlaneRows al{x.p, ldx, x_batch_stride, x.stride}, bl{w.p, K, 0, w.stride};
    if (out_planes.p) {
        if (out_planes.count == 3)
            launch_linear_planes(s, M, N, K, batches, al, bl, 3,
                                 EpGeluPlanes<3>{out_planes.p, bias, ldo, obs, out_planes.stride});
        else
            launch_linear_planes(s, M, N, K, batches, al, bl, 1,
                                 EpGeluPlanes<1>{out_planes.p, bias, ldo, obs, out_planes.stride});
        return;
    }
    EpLinear ep;
    ep.out = out;
    ep.bias = bias;
    ep.residual = residual;
    ep.gamma = gamma;
    ep.stats = stats;
    ep.ldo = ldo;
    ep.batch_stride = obs;
    ep.tail = tail;
    launch_linear_planes(s, M, N, K, batches, al, bl, x.count, ep);
}

void linear_qkv_planes(hipStream_t s, Planes x, int64_t ldx, int64_t x_batch_stride, Planes w, const float *bias,
                       int batches, int M, int K, int N, int q_cols, float *q, const KVPlanes &kv) {
    require_ptrs({x.p, w.p, bias, kv.k, kv.vt}, "linear_qkv_planes");
    DMX_REQUIRE(x.count == 3 && w.count == 3, "linear_qkv_planes: three planes");
    DMX_REQUIRE(q_cols == 0 || q, "linear_qkv_planes: q output missing");
    const int D = (N - q_cols) / 2;
    DMX_REQUIRE(D > 0 && D % 64 == 0 && (q_cols == 0 || q_cols == D) && q_cols + 2 * D == N,
                "linear_qkv_planes: columns must be [q |] k | v with D a multiple of 64");
    DMX_REQUIRE(kv.ldk >= D && kv.ldvt >= kv_ldvt(M) && kv.ldvt % 32 == 0 && kv.k_stride % 4 == 0 &&
                    kv.k_bs % 4 == 0 && kv.ldk % 4 == 0 && kv.vt_stride % 4 == 0 &&
                    ((reinterpret_cast<uintptr_t>(kv.k) | reinterpret_cast<uintptr_t>(kv.vt)) & 7) == 0,
                "linear_qkv_planes: K/V planes layout");
    EpQKV ep;
    ep.q = q;
    ep.q_bs = (int64_t)M * D;
    ep.bias = bias;
    ep.kv = kv;
    ep.q_cols = q_cols;
    ep.D = D;
    launch_linear_planes(s, M, N, K, batches, PlaneRows{x.p, ldx, x_batch_stride, x.stride},
                         PlaneRows{w.p, K, 0, w.stride}, 3, ep);
}

void tokens_to_channels(hipStream_t s, const float *tok, int b, int F, int T, int D, const float *w, const float *bias,
                        int M, float *out) {
    require_ptrs({tok, w, out}, "tokens_to_channels");
    DMX_REQUIRE(D % 4 == 0 && aligned16(tok), "tokens_to_channels: token rows must be float4 aligned");
    EpChannels ep;
    ep.out = out;
    ep.bias = bias;
    ep.batch_stride = (int64_t)M * F * T;
    ep.N = F * T;
    ep.act = ACT_NONE;
    ep.vec = !ep.bias || aligned16(ep.bias);
    // A rearrange (w is the identity in the transformer-only path): kept in
    // fp32 whatever the precision scope, so it stays exact.
    gemm_pick<false, false>(s, M, F * T, D, b, kmajor(w, D, 0), TokenGather{tok, F, T, D}, ep);
}

}  // namespace dmx
