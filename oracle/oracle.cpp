// oracle.cpp — CPU restatement of eclipse005/demucs-wgpu's host (CPU) backend.
//
// TEST INFRASTRUCTURE ONLY: the parity checker and the timed CPU baseline. The
// product library never links or calls this file.
//
// Every function cites the reference function it restates
// (paths relative to /root/reference/crates/demucs-core/src). The arithmetic
// follows the reference: f32 GEMM accumulation, f64 moments for GroupNorm and
// the input/global normalisation, f32 two-pass LayerNorm, the rational erfc
// GELU, the deferred-division softmax. Where the reference delegates to a
// third-party crate the published algorithm is restated:
//   * gemm 0.18.2 (Cargo.lock): C = A.B with f32 accumulation;
//   * rustfft 6.4.1 (Cargo.lock): the DFT X[k] = sum_n x[n] e^{-+2 pi i kn/N},
//     unnormalised both ways; computed here in f64 and rounded to f32.
// Summation order inside a GEMM / FFT differs from those crates; the values
// agree to f32 rounding.

#include "oracle.h"

#include <omp.h>

#include <algorithm>
#include <functional>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

thread_local std::string g_error;

struct OracleError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

[[noreturn]] void fail(const std::string &msg) { throw OracleError(msg); }

template <class F>
int guarded(F &&f) {
    try {
        f();
        g_error.clear();
        return 0;
    } catch (const std::exception &e) {
        g_error = e.what();
        return 1;
    }
}

constexpr double kPi = 3.14159265358979323846;

typedef float v8f __attribute__((vector_size(32)));

// ---------------------------------------------------------------------------
// GEMM (the `gemm` crate's role: demucs/ops.rs:807-839, 1110-1152).
// C[m x n] = A[m x k] . B[k x n], any strides, f32 accumulation, overwrite.
// Packed, cache-blocked; a 6x16 register micro-kernel on GCC vector types.
// ---------------------------------------------------------------------------
constexpr int64_t MR = 6, NR = 16, KC = 256, MC = 72, NC = 512;

void pack_a(const float *a, int64_t a_rs, int64_t a_cs, int64_t m0, int64_t mc, int64_t k0,
            int64_t kc, float *dst) {
    for (int64_t i = 0; i < mc; i += MR) {
        int64_t rows = std::min(MR, mc - i);
        for (int64_t p = 0; p < kc; ++p) {
            for (int64_t r = 0; r < MR; ++r)
                dst[r] = r < rows ? a[(m0 + i + r) * a_rs + (k0 + p) * a_cs] : 0.0f;
            dst += MR;
        }
    }
}

void pack_b(const float *b, int64_t b_rs, int64_t b_cs, int64_t k0, int64_t kc, int64_t n0,
            int64_t nc, float *dst) {
    for (int64_t j = 0; j < nc; j += NR) {
        int64_t cols = std::min(NR, nc - j);
        for (int64_t p = 0; p < kc; ++p) {
            const float *src = b + (k0 + p) * b_rs + (n0 + j) * b_cs;
            if (cols == NR && b_cs == 1) {
                std::memcpy(dst, src, NR * sizeof(float));
            } else {
                for (int64_t c = 0; c < NR; ++c) dst[c] = c < cols ? src[c * b_cs] : 0.0f;
            }
            dst += NR;
        }
    }
}

// acc(MR x NR) (+)= Apanel(MR x kc) . Bpanel(kc x NR)
inline void micro_kernel(int64_t kc, const float *ap, const float *bp, float *c, int64_t ldc,
                         int64_t rows, int64_t cols, bool accumulate) {
    v8f acc[MR][2];
    for (int r = 0; r < MR; ++r) acc[r][0] = acc[r][1] = (v8f){0, 0, 0, 0, 0, 0, 0, 0};
    for (int64_t p = 0; p < kc; ++p) {
        v8f b0, b1;
        std::memcpy(&b0, bp, 32);
        std::memcpy(&b1, bp + 8, 32);
        for (int r = 0; r < MR; ++r) {
            v8f a = (v8f){ap[r], ap[r], ap[r], ap[r], ap[r], ap[r], ap[r], ap[r]};
            acc[r][0] += a * b0;
            acc[r][1] += a * b1;
        }
        ap += MR;
        bp += NR;
    }
    float tmp[NR];
    for (int64_t r = 0; r < rows; ++r) {
        std::memcpy(tmp, &acc[r][0], 32);
        std::memcpy(tmp + 8, &acc[r][1], 32);
        float *row = c + r * ldc;
        if (accumulate)
            for (int64_t j = 0; j < cols; ++j) row[j] += tmp[j];
        else
            for (int64_t j = 0; j < cols; ++j) row[j] = tmp[j];
    }
}

void sgemm(int64_t m, int64_t n, int64_t k, const float *a, int64_t a_rs, int64_t a_cs,
           const float *b, int64_t b_rs, int64_t b_cs, float *c, int64_t ldc) {
    if (m <= 0 || n <= 0) return;
    if (k <= 0) {
        for (int64_t i = 0; i < m; ++i) std::fill(c + i * ldc, c + i * ldc + n, 0.0f);
        return;
    }
    const bool nested = omp_in_parallel();
    // Parallel over (m-block, n-block) tiles; every tile runs the whole k loop,
    // so no two threads ever write the same element.
    int64_t m_blocks = (m + MC - 1) / MC, n_blocks = (n + NC - 1) / NC;
    int64_t tiles = m_blocks * n_blocks;
#pragma omp parallel for schedule(dynamic) if (!nested && tiles > 1 && m * n * k > 32768)
    for (int64_t t = 0; t < tiles; ++t) {
        int64_t mb = t / n_blocks, nb = t % n_blocks;
        int64_t m0 = mb * MC, mc = std::min(MC, m - m0);
        int64_t n0 = nb * NC, nc = std::min(NC, n - n0);
        std::vector<float> apack(((mc + MR - 1) / MR) * MR * KC);
        std::vector<float> bpack(((nc + NR - 1) / NR) * NR * KC);
        for (int64_t k0 = 0; k0 < k; k0 += KC) {
            int64_t kc = std::min(KC, k - k0);
            pack_a(a, a_rs, a_cs, m0, mc, k0, kc, apack.data());
            pack_b(b, b_rs, b_cs, k0, kc, n0, nc, bpack.data());
            for (int64_t j = 0; j < nc; j += NR) {
                for (int64_t i = 0; i < mc; i += MR) {
                    micro_kernel(kc, apack.data() + (i / MR) * MR * kc,
                                 bpack.data() + (j / NR) * NR * kc, c + (m0 + i) * ldc + n0 + j, ldc,
                                 std::min(MR, mc - i), std::min(NR, nc - j), k0 > 0);
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Pointwise (ops.rs:95-121, demucs/ops.rs:624-663)
// ---------------------------------------------------------------------------

// `erf` of ops.rs:101-121: erfc by the Numerical Recipes rational
// approximation (Press et al., "erfcc", fractional error < 1.2e-7).
inline float erf_nr(float x) {
    float z = std::fabs(x);
    float t = 1.0f / (1.0f + 0.5f * z);
    float poly =
        -z * z - 1.26551223f +
        t * (1.00002368f +
             t * (0.37409196f +
                  t * (0.09678418f +
                       t * (-0.18628806f +
                            t * (0.27886807f +
                                 t * (-1.13520398f +
                                      t * (1.48851587f + t * (-0.82215223f + t * 0.17087277f))))))));
    float tau = t * std::exp(poly);
    float value = 1.0f - tau;
    return x >= 0.0f ? value : -value;
}

// `gelu_erf` (ops.rs:95-97).
inline float gelu(float x) { return 0.5f * x * (1.0f + erf_nr(x * 0.70710678118654752440f)); }

inline float sigmoid_ref(float g) { return 1.0f / (1.0f + std::exp(-g)); }

void gelu_inplace(float *x, int64_t n) {
#pragma omp parallel for schedule(static) if (!omp_in_parallel() && n > 65536)
    for (int64_t i = 0; i < n; ++i) x[i] = gelu(x[i]);
}

// ---------------------------------------------------------------------------
// Convolutions (demucs/ops.rs:44-211, 366-405, 414-528)
// ---------------------------------------------------------------------------

// `conv2d` (demucs/ops.rs:44-211): im2col over output positions + one GEMM
// (oc, k) x (k, positions) + bias; a 1x1/stride-1/unpadded kernel is the GEMM
// on the input directly (demucs/ops.rs:78-115).
void conv2d(const float *x, int64_t batch, int64_t ic, int64_t h, int64_t w, const float *weight,
            const float *bias, int64_t oc, int64_t kh, int64_t kw, int64_t sh, int64_t sw,
            int64_t ph, int64_t pw, int64_t dh, int64_t dw, float *out) {
    int64_t eh = dh * (kh - 1) + 1, ew = dw * (kw - 1) + 1;
    if (h + 2 * ph < eh || w + 2 * pw < ew) fail("conv2d: kernel larger than the padded input");
    int64_t oh = (h + 2 * ph - eh) / sh + 1, ow = (w + 2 * pw - ew) / sw + 1;
    int64_t k = ic * kh * kw, plane = oh * ow;
    const bool pointwise = kh == 1 && kw == 1 && sh == 1 && sw == 1 && ph == 0 && pw == 0;
    std::vector<float> patches;
    for (int64_t bi = 0; bi < batch; ++bi) {
        const float *src = x + bi * ic * h * w;
        float *dst = out + bi * oc * plane;
        const float *cols = src;
        if (!pointwise) {
            patches.resize(k * plane);
#pragma omp parallel for schedule(static) if (!omp_in_parallel())
            for (int64_t row = 0; row < k; ++row) {
                int64_t c = row / (kh * kw), tap = row % (kh * kw), ky = tap / kw, kx = tap % kw;
                float *prow = patches.data() + row * plane;
                for (int64_t oy = 0; oy < oh; ++oy) {
                    int64_t iy = oy * sh + ky * dh - ph;
                    for (int64_t ox = 0; ox < ow; ++ox) {
                        int64_t ix = ox * sw + kx * dw - pw;
                        prow[oy * ow + ox] = (iy < 0 || iy >= h || ix < 0 || ix >= w)
                                                 ? 0.0f
                                                 : src[(c * h + iy) * w + ix];
                    }
                }
            }
            cols = patches.data();
        }
        sgemm(oc, plane, k, weight, k, 1, cols, plane, 1, dst, plane);
#pragma omp parallel for schedule(static) if (!omp_in_parallel())
        for (int64_t o = 0; o < oc; ++o) {
            float shift = bias ? bias[o] : 0.0f;
            if (shift != 0.0f)
                for (int64_t p = 0; p < plane; ++p) dst[o * plane + p] += shift;
        }
    }
}

// `conv_transpose2d` (demucs/ops.rs:414-515): no padding, no output padding;
// bias first, then the taps in (ky, kx) order, one stacked GEMM
// (kh*kw*oc, ic) x (ic, positions).
void conv_transpose2d(const float *x, int64_t batch, int64_t ic, int64_t h, int64_t w,
                      const float *weight, const float *bias, int64_t oc, int64_t kh, int64_t kw,
                      int64_t sh, int64_t sw, float *out) {
    int64_t oh = (h - 1) * sh + kh, ow = (w - 1) * sw + kw, positions = h * w;
    std::vector<float> taps(kh * kw * oc * ic);
    for (int64_t ky = 0; ky < kh; ++ky)
        for (int64_t kx = 0; kx < kw; ++kx)
            for (int64_t c = 0; c < ic; ++c)
                for (int64_t o = 0; o < oc; ++o)
                    taps[((ky * kw + kx) * oc + o) * ic + c] = weight[((c * oc + o) * kh + ky) * kw + kx];
    std::vector<float> product(kh * kw * oc * positions);
    for (int64_t bi = 0; bi < batch; ++bi) {
        sgemm(kh * kw * oc, positions, ic, taps.data(), ic, 1, x + bi * ic * positions, positions,
              1, product.data(), positions);
        float *plane = out + bi * oc * oh * ow;
#pragma omp parallel for schedule(static) if (!omp_in_parallel())
        for (int64_t o = 0; o < oc; ++o) {
            float *target = plane + o * oh * ow;
            std::fill(target, target + oh * ow, bias ? bias[o] : 0.0f);
            for (int64_t tap = 0; tap < kh * kw; ++tap) {
                int64_t ky = tap / kw, kx = tap % kw;
                const float *source = product.data() + (tap * oc + o) * positions;
                for (int64_t iy = 0; iy < h; ++iy)
                    for (int64_t ix = 0; ix < w; ++ix)
                        target[(iy * sh + ky) * ow + ix * sw + kx] += source[iy * w + ix];
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Norms (demucs/ops.rs:532-621, 674-743; host.rs:1137-1196)
// ---------------------------------------------------------------------------

struct Moments {
    float mean;
    float inv;
};

// f64 sum / sum of squares of a run, then the reference's mean and
// 1/sqrt(var + 1e-5) with the sqrt in f64 and the reciprocal in f32
// (demucs/ops.rs:568-579).
Moments moments_f64(const float *x, int64_t n) {
    double sum = 0.0, sum_sq = 0.0;
    for (int64_t i = 0; i < n; ++i) {
        double v = x[i];
        sum += v;
        sum_sq += v * v;
    }
    double count = (double)n, mean = sum / count;
    double variance = std::max(sum_sq / count - mean * mean, 0.0);
    return {(float)mean, 1.0f / (float)std::sqrt(variance + 1e-5)};
}

// `group_norm` (demucs/ops.rs:532-593).
void group_norm(const float *x, int64_t batch, int64_t channels, int64_t inner, int64_t groups,
                const float *weight, const float *bias, float *out) {
    if (groups <= 0 || channels % groups) fail("group_norm: channels not divisible by groups");
    int64_t per_group = channels / groups, pairs = batch * groups, len = per_group * inner;
#pragma omp parallel for schedule(dynamic) if (!omp_in_parallel())
    for (int64_t pair = 0; pair < pairs; ++pair) {
        int64_t g = pair % groups;
        const float *src = x + pair * len;
        float *dst = out + pair * len;
        Moments mo = moments_f64(src, len);
        for (int64_t c = 0; c < per_group; ++c) {
            float scale = mo.inv * weight[g * per_group + c];
            float shift = bias[g * per_group + c] - mo.mean * scale;
            for (int64_t i = 0; i < inner; ++i) dst[c * inner + i] = src[c * inner + i] * scale + shift;
        }
    }
}

// `group_norm_glu` (demucs/ops.rs:674-743): same statistics, then a*sigmoid(g).
void group_norm_glu(const float *x, int64_t batch, int64_t channels, int64_t inner, int64_t groups,
                    const float *weight, const float *bias, float *out) {
    if (groups <= 0 || channels % groups) fail("group_norm_glu: channels not divisible");
    int64_t per_group = channels / groups;
    if (per_group % 2) fail("group_norm_glu needs an even per-group channel count");
    int64_t half = per_group / 2, pairs = batch * groups;
#pragma omp parallel for schedule(dynamic) if (!omp_in_parallel())
    for (int64_t pair = 0; pair < pairs; ++pair) {
        int64_t g = pair % groups;
        const float *chunk = x + pair * per_group * inner;
        float *dst = out + pair * half * inner;
        Moments mo = moments_f64(chunk, per_group * inner);
        for (int64_t c = 0; c < half; ++c) {
            float vs = mo.inv * weight[g * per_group + c];
            float vsh = bias[g * per_group + c] - mo.mean * vs;
            float gs = mo.inv * weight[g * per_group + c + half];
            float gsh = bias[g * per_group + c + half] - mo.mean * gs;
            for (int64_t i = 0; i < inner; ++i) {
                float value = chunk[c * inner + i] * vs + vsh;
                float gate = chunk[(c + half) * inner + i] * gs + gsh;
                dst[c * inner + i] = value * sigmoid_ref(gate);
            }
        }
    }
}

// `layer_norm_rows` (demucs/ops.rs:596-621): f32 two-pass per row.
void layer_norm_rows(const float *x, int64_t rows, int64_t dim, const float *weight,
                     const float *bias, float *out) {
#pragma omp parallel for schedule(static) if (!omp_in_parallel() && rows > 16)
    for (int64_t r = 0; r < rows; ++r) {
        const float *row = x + r * dim;
        float sum = 0.0f;
        for (int64_t i = 0; i < dim; ++i) sum += row[i];
        float mean = sum / (float)dim;
        float var = 0.0f;
        for (int64_t i = 0; i < dim; ++i) var += (row[i] - mean) * (row[i] - mean);
        var /= (float)dim;
        float inv = 1.0f / std::sqrt(var + 1e-5f);
        for (int64_t i = 0; i < dim; ++i) out[r * dim + i] = (row[i] - mean) * inv * weight[i] + bias[i];
    }
}

// `group_norm_positions` (host.rs:1137-1196): MyGroupNorm(1, C) on (b, t, c),
// statistics over the whole (t, c) plane in 32 K-element f64 blocks combined in order.
void group_norm_positions(float *x, int64_t batch, int64_t t, int64_t c, const float *weight,
                          const float *bias) {
    int64_t plane = t * c;
    for (int64_t bi = 0; bi < batch; ++bi) {
        float *p = x + bi * plane;
        int64_t blocks = (plane + 32767) / 32768;
        std::vector<double> bs(blocks), bq(blocks);
#pragma omp parallel for schedule(static) if (!omp_in_parallel())
        for (int64_t blk = 0; blk < blocks; ++blk) {
            double s = 0.0, q = 0.0;
            for (int64_t i = blk * 32768; i < std::min(plane, (blk + 1) * 32768); ++i) {
                double v = p[i];
                s += v;
                q += v * v;
            }
            bs[blk] = s;
            bq[blk] = q;
        }
        double sum = 0.0, sum_sq = 0.0;
        for (int64_t blk = 0; blk < blocks; ++blk) {
            sum += bs[blk];
            sum_sq += bq[blk];
        }
        double count = (double)plane, mean = sum / count;
        double variance = std::max(sum_sq / count - mean * mean, 0.0);
        float inv = 1.0f / (float)std::sqrt(variance + 1e-5);
        float meanf = (float)mean;
        std::vector<float> scale(c), shift(c);
        for (int64_t ch = 0; ch < c; ++ch) {
            scale[ch] = inv * weight[ch];
            shift[ch] = bias[ch] - meanf * scale[ch];
        }
#pragma omp parallel for schedule(static) if (!omp_in_parallel())
        for (int64_t row = 0; row < t; ++row)
            for (int64_t ch = 0; ch < c; ++ch) p[row * c + ch] = p[row * c + ch] * scale[ch] + shift[ch];
    }
}

// `glu` (demucs/ops.rs:624-658) on (b, 2c, inner).
void glu(const float *x, int64_t batch, int64_t channels, int64_t inner, float *out) {
    if (channels % 2) fail("GLU needs an even channel count");
    int64_t half = channels / 2;
#pragma omp parallel for schedule(static) if (!omp_in_parallel())
    for (int64_t row = 0; row < batch * half; ++row) {
        int64_t bi = row / half, c = row % half;
        const float *value = x + (bi * channels + c) * inner;
        const float *gate = value + half * inner;
        for (int64_t i = 0; i < inner; ++i) out[row * inner + i] = value[i] * sigmoid_ref(gate[i]);
    }
}

// `std_unbiased` / `mean` (demucs/ops.rs:1494-1509, 1585-1590).
float std_unbiased(const float *x, int64_t n) {
    if (n < 2) return NAN;
    double mean = 0.0;
    for (int64_t i = 0; i < n; ++i) mean += x[i];
    mean /= (double)n;
    double var = 0.0;
    for (int64_t i = 0; i < n; ++i) {
        double d = (double)x[i] - mean;
        var += d * d;
    }
    return (float)std::sqrt(var / (double)(n - 1));
}

float mean_f64(const float *x, int64_t n) {
    if (n == 0) return NAN;
    double s = 0.0;
    for (int64_t i = 0; i < n; ++i) s += x[i];
    return (float)(s / (double)n);
}

// ---------------------------------------------------------------------------
// Attention (demucs/ops.rs:1350-1458, host.rs:1199-1312)
// ---------------------------------------------------------------------------

// `attention_head` with the deferred softmax division (demucs/ops.rs:1350-1400,
// 1442-1458): S = (q*scale) k^T; P = exp(S - rowmax); O = P v; O /= rowsum.
void attention_head(const float *q, int64_t q_rs, const float *k, int64_t k_rs, const float *v,
                    int64_t v_rs, int64_t n_q, int64_t n_k, int64_t d, float scale, float *out,
                    int64_t out_rs) {
    std::vector<float> scaled(n_q * d), scores(n_q * n_k), o(n_q * d);
    for (int64_t i = 0; i < n_q; ++i)
        for (int64_t j = 0; j < d; ++j) scaled[i * d + j] = q[i * q_rs + j] * scale;
    sgemm(n_q, n_k, d, scaled.data(), d, 1, k, 1, k_rs, scores.data(), n_k);
    std::vector<float> sums(n_q);
    for (int64_t i = 0; i < n_q; ++i) {
        float *row = scores.data() + i * n_k;
        float mx = -INFINITY;
        for (int64_t j = 0; j < n_k; ++j) mx = std::max(mx, row[j]);
        float sum = 0.0f;
        for (int64_t j = 0; j < n_k; ++j) {
            row[j] = std::exp(row[j] - mx);
            sum += row[j];
        }
        sums[i] = sum;
    }
    sgemm(n_q, d, n_k, scores.data(), n_k, 1, v, v_rs, 1, o.data(), d);
    for (int64_t i = 0; i < n_q; ++i) {
        float inv = sums[i] > 0.0f ? 1.0f / sums[i] : 1.0f;
        for (int64_t j = 0; j < d; ++j) out[i * out_rs + j] = sums[i] > 0.0f ? o[i * d + j] * inv : o[i * d + j];
    }
}

// `Linear::forward` (ops.rs:16-63, demucs/ops.rs:1191-1216): x (rows, in)
// . W^T (W stored (out, in)) + bias.
void linear(const float *x, int64_t rows, int64_t in, const float *w, const float *b, int64_t out_f,
            float *out) {
    sgemm(rows, out_f, in, x, in, 1, w, 1, in, out, out_f);
    if (b) {
#pragma omp parallel for schedule(static) if (!omp_in_parallel() && rows > 64)
        for (int64_t r = 0; r < rows; ++r)
            for (int64_t j = 0; j < out_f; ++j) out[r * out_f + j] += b[j];
    }
}

// `multi_head_attention` (host.rs:1199-1312).
void multi_head_attention(const float *query, const float *key, int64_t batch, int64_t n_q,
                          int64_t n_k, int64_t dim, int64_t heads, const float *wq, const float *bq,
                          const float *wk, const float *bk, const float *wv, const float *bv,
                          const float *wo, const float *bo, float *out,
                          std::vector<float> *q_out = nullptr, std::vector<float> *k_out = nullptr,
                          std::vector<float> *v_out = nullptr) {
    int64_t dh = dim / heads;
    float scale = 1.0f / std::sqrt((float)dh);
    std::vector<float> q(batch * n_q * dim), k(batch * n_k * dim), v(batch * n_k * dim),
        merged(batch * n_q * dim);
    linear(query, batch * n_q, dim, wq, bq, dim, q.data());
    linear(key, batch * n_k, dim, wk, bk, dim, k.data());
    linear(key, batch * n_k, dim, wv, bv, dim, v.data());
#pragma omp parallel for schedule(dynamic) if (!omp_in_parallel())
    for (int64_t bh = 0; bh < batch * heads; ++bh) {
        int64_t bi = bh / heads, h = bh % heads;
        attention_head(q.data() + bi * n_q * dim + h * dh, dim, k.data() + bi * n_k * dim + h * dh,
                       dim, v.data() + bi * n_k * dim + h * dh, dim, n_q, n_k, dh, scale,
                       merged.data() + bi * n_q * dim + h * dh, dim);
    }
    linear(merged.data(), batch * n_q, dim, wo, bo, dim, out);
    if (q_out) *q_out = std::move(q);
    if (k_out) *k_out = std::move(k);
    if (v_out) *v_out = std::move(v);
}

// ---------------------------------------------------------------------------
// STFT (dsp/stft.rs:54-326) and HTDemucs framing (demucs/spec.rs)
// ---------------------------------------------------------------------------

// Periodic Hann (stft.rs:54-61).
std::vector<float> hann(int64_t n) {
    std::vector<float> w(n);
    for (int64_t i = 0; i < n; ++i) {
        double phase = 2.0 * kPi * (double)i / (double)n;
        w[i] = (float)(0.5 - 0.5 * std::cos(phase));
    }
    return w;
}

// In-place complex DFT in f64: radix-2 for powers of two, direct otherwise.
// sign = -1 forward, +1 inverse, unnormalised (rustfft's convention).
void dft(std::vector<double> &re, std::vector<double> &im, int sign) {
    size_t n = re.size();
    if (n == 0) return;
    if ((n & (n - 1)) != 0) {
        std::vector<double> orr(n), oi(n);
        for (size_t kk = 0; kk < n; ++kk) {
            double sr = 0, si = 0;
            for (size_t t = 0; t < n; ++t) {
                double ang = sign * 2.0 * kPi * (double)((kk * t) % n) / (double)n;
                sr += re[t] * std::cos(ang) - im[t] * std::sin(ang);
                si += re[t] * std::sin(ang) + im[t] * std::cos(ang);
            }
            orr[kk] = sr;
            oi[kk] = si;
        }
        re.swap(orr);
        im.swap(oi);
        return;
    }
    for (size_t i = 1, j = 0; i < n; ++i) {
        size_t bit = n >> 1;
        for (; j & bit; bit >>= 1) j ^= bit;
        j ^= bit;
        if (i < j) {
            std::swap(re[i], re[j]);
            std::swap(im[i], im[j]);
        }
    }
    for (size_t len = 2; len <= n; len <<= 1) {
        size_t half = len / 2;
        for (size_t j = 0; j < half; ++j) {
            double ang = sign * 2.0 * kPi * (double)j / (double)len;
            double wr = std::cos(ang), wi = std::sin(ang);
            for (size_t i = 0; i < n; i += len) {
                double ur = re[i + j], ui = im[i + j];
                double vr = re[i + j + half] * wr - im[i + j + half] * wi;
                double vi = re[i + j + half] * wi + im[i + j + half] * wr;
                re[i + j] = ur + vr;
                im[i + j] = ui + vi;
                re[i + j + half] = ur - vr;
                im[i + j + half] = ui - vi;
            }
        }
    }
}

// `pad_signal` reflect (stft.rs:310-326).
std::vector<float> reflect_center(const float *s, int64_t len, int64_t pad) {
    std::vector<float> out(len + 2 * pad, 0.0f);
    std::memcpy(out.data() + pad, s, len * sizeof(float));
    for (int64_t i = 0; i < pad; ++i) {
        out[pad - 1 - i] = s[i + 1];
        out[pad + len + i] = s[len - 2 - i];
    }
    return out;
}

// `Stft::forward` (stft.rs:126-201), center=True, reflect, win = n_fft.
int64_t stft(const float *x, int64_t batch, int64_t samples, int64_t n_fft, int64_t hop,
             bool normalized, float *out_re, float *out_im) {
    int64_t pad = n_fft / 2;
    if (pad >= samples) fail("reflect padding needs an input longer than n_fft/2");
    int64_t frames = 1 + (samples + n_fft - n_fft) / hop;
    int64_t bins = n_fft / 2 + 1;
    float norm_scale = normalized ? 1.0f / std::sqrt((float)n_fft) : 1.0f;
    std::vector<float> window = hann(n_fft);
    for (int64_t b = 0; b < batch; ++b) {
        std::vector<float> row = reflect_center(x + b * samples, samples, pad);
#pragma omp parallel for schedule(static) if (!omp_in_parallel())
        for (int64_t f = 0; f < frames; ++f) {
            std::vector<double> re(n_fft), im(n_fft, 0.0);
            for (int64_t i = 0; i < n_fft; ++i) re[i] = (double)(row[f * hop + i] * window[i]);
            dft(re, im, -1);
            for (int64_t k = 0; k < bins; ++k) {
                out_re[(b * bins + k) * frames + f] = (float)re[k] * norm_scale;
                out_im[(b * bins + k) * frames + f] = (float)im[k] * norm_scale;
            }
        }
    }
    return frames;
}

// `Stft::inverse` (stft.rs:204-295). length < 0 means None.
int64_t istft(const float *re, const float *im, int64_t batch, int64_t bins, int64_t frames,
              int64_t n_fft, int64_t hop, bool normalized, int64_t length, float *out) {
    if (bins != n_fft / 2 + 1) fail("istft: bin count does not match n_fft");
    if (frames == 0) fail("cannot invert an empty spectrogram");
    int64_t expected = n_fft + hop * (frames - 1);
    int64_t start = n_fft / 2;
    int64_t end = length >= 0 ? start + length : expected - n_fft / 2;
    end = std::min(end, expected);
    int64_t out_len = std::max<int64_t>(end - start, 0);
    float norm_scale = normalized ? std::sqrt((float)n_fft) : 1.0f;
    float inv_n = norm_scale / (float)n_fft;
    std::vector<float> window = hann(n_fft);
    if (!out) return out_len;
#pragma omp parallel for schedule(dynamic) if (!omp_in_parallel())
    for (int64_t b = 0; b < batch; ++b) {
        std::vector<float> y(expected, 0.0f), env(expected, 0.0f);
        std::vector<double> br(n_fft), bim(n_fft);
        for (int64_t f = 0; f < frames; ++f) {
            br[0] = re[(b * bins + 0) * frames + f];
            bim[0] = im[(b * bins + 0) * frames + f];
            for (int64_t k = 1; k < bins; ++k) {
                double r = re[(b * bins + k) * frames + f], i = im[(b * bins + k) * frames + f];
                br[k] = r;
                bim[k] = i;
                br[n_fft - k] = r;
                bim[n_fft - k] = -i;
            }
            std::vector<double> xr(br), xi(bim);
            dft(xr, xi, +1);
            int64_t offset = f * hop;
            for (int64_t i = 0; i < n_fft; ++i) {
                float w = window[i];
                y[offset + i] += (float)xr[i] * inv_n * w;
                env[offset + i] += w * w;
            }
        }
        for (int64_t i = start; i < end; ++i) out[b * out_len + i - start] = env[i] != 0.0f ? y[i] / env[i] : 0.0f;
    }
    return out_len;
}

// `pad1d_reflect` (demucs/spec.rs:204-236), with hdemucs.py's short-input fallback.
std::vector<float> pad1d_reflect(const float *x, int64_t length, int64_t left, int64_t right) {
    int64_t max_pad = std::max(left, right), extra_left = 0, extra_right = 0;
    if (length <= max_pad) {
        int64_t extra = max_pad - length + 1;
        extra_right = std::min(right, extra);
        extra_left = extra - extra_right;
    }
    int64_t pl = left - extra_left, pr = right - extra_right;
    std::vector<float> base(extra_left, 0.0f);
    base.insert(base.end(), x, x + length);
    base.insert(base.end(), extra_right, 0.0f);
    int64_t bl = (int64_t)base.size();
    if (bl <= pl || bl <= pr) fail("reflect padding needs more samples");
    std::vector<float> out(bl + pl + pr, 0.0f);
    std::copy(base.begin(), base.end(), out.begin() + pl);
    for (int64_t i = 0; i < pl; ++i) out[pl - 1 - i] = base[i + 1];
    for (int64_t i = 0; i < pr; ++i) out[pl + bl + i] = base[bl - 2 - i];
    return out;
}

// `DemucsSpec::spec` (demucs/spec.rs:62-113) followed by
// `pack_complex_as_channels` (demucs/spec.rs:240-254).
void spec_cac(const float *mix, int64_t batch, int64_t channels, int64_t length, int64_t nfft,
              float *out) {
    int64_t hl = nfft / 4, le = (length + hl - 1) / hl, pad = hl / 2 * 3;
    int64_t right = pad + le * hl - length, padded_len = length + pad + right;
    int64_t bins = nfft / 2 + 1;
    std::vector<float> padded(batch * channels * padded_len);
    for (int64_t r = 0; r < batch * channels; ++r) {
        std::vector<float> v = pad1d_reflect(mix + r * length, length, pad, right);
        std::copy(v.begin(), v.end(), padded.begin() + r * padded_len);
    }
    int64_t frames = 1 + padded_len / hl;
    if (frames != le + 4) fail("spectro produced an unexpected frame count");
    std::vector<float> re(batch * channels * bins * frames), im(re.size());
    stft(padded.data(), batch * channels, padded_len, nfft, hl, true, re.data(), im.data());
    int64_t fr = bins - 1;
    for (int64_t b = 0; b < batch; ++b)
        for (int64_t c = 0; c < channels; ++c)
            for (int64_t f = 0; f < fr; ++f)
                for (int64_t t = 0; t < le; ++t) {
                    int64_t src = ((b * channels + c) * bins + f) * frames + t + 2;
                    out[((b * 2 * channels + 2 * c) * fr + f) * le + t] = re[src];
                    out[((b * 2 * channels + 2 * c + 1) * fr + f) * le + t] = im[src];
                }
}

// `unpack_channels_as_complex` + `pad_for_ispec` + `DemucsSpec::ispec`
// (demucs/spec.rs:268-340, 117-175): x (b, 4s, fr, le) with channels
// s*4 + c*2 + {0: re, 1: im}; returns (b, s, 2, length).
void ispec_cac(const float *x, int64_t batch, int64_t sources, int64_t fr, int64_t le, int64_t nfft,
               int64_t length, float *out) {
    int64_t hop = nfft / 4, pad = hop / 2 * 3;
    int64_t bins = fr + 1, frames = le + 4;
    if (2 * bins - 2 != nfft) fail("_ispec: bin count does not imply nfft");
    int64_t total = hop * ((length + hop - 1) / hop) + 2 * pad;
    int64_t rows = batch * sources * 2;
    std::vector<float> re(rows * bins * frames, 0.0f), im(rows * bins * frames, 0.0f);
    for (int64_t r = 0; r < rows; ++r) {
        int64_t b = r / (sources * 2), s = (r / 2) % sources, c = r % 2;
        const float *real = x + ((b * sources * 4) + s * 4 + c * 2) * fr * le;
        const float *imag = real + fr * le;
        for (int64_t f = 0; f < fr; ++f)
            for (int64_t t = 0; t < le; ++t) {
                re[(r * bins + f) * frames + t + 2] = real[f * le + t];
                im[(r * bins + f) * frames + t + 2] = imag[f * le + t];
            }
    }
    int64_t out_len = istft(re.data(), im.data(), rows, bins, frames, nfft, hop, true, total, nullptr);
    std::vector<float> rebuilt(rows * out_len);
    istft(re.data(), im.data(), rows, bins, frames, nfft, hop, true, total, rebuilt.data());
    if (out_len < pad + length) fail("istft produced too few samples");
    for (int64_t r = 0; r < rows; ++r)
        std::memcpy(out + r * length, rebuilt.data() + r * out_len + pad, length * sizeof(float));
}

// `two_dimensional_positions` (host.rs:1078-1106).
void positions_2d(int64_t dim, int64_t height, int64_t width, float max_period, float *out) {
    int64_t half = dim / 2, pairs = half / 2;
    float log_period = std::log(max_period) / (float)half;
    std::vector<float> div(pairs);
    for (int64_t j = 0; j < pairs; ++j) div[j] = std::exp(-(float)(2 * j) * log_period);
    for (int64_t t = 0; t < width; ++t)
        for (int64_t f = 0; f < height; ++f) {
            float *tok = out + (t * height + f) * dim;
            for (int64_t j = 0; j < pairs; ++j) {
                float w = (float)t * div[j], h = (float)f * div[j];
                tok[2 * j] = std::sin(w);
                tok[2 * j + 1] = std::cos(w);
                tok[half + 2 * j] = std::sin(h);
                tok[half + 2 * j + 1] = std::cos(h);
            }
        }
}

// `one_dimensional_positions` (host.rs:1110-1122).
void positions_1d(int64_t length, int64_t dim, float max_period, float *out) {
    int64_t half = dim / 2;
    for (int64_t t = 0; t < length; ++t)
        for (int64_t i = 0; i < half; ++i) {
            float exponent = (float)i / ((float)half - 1.0f);
            float phase = (float)t / std::pow(max_period, exponent);
            out[t * dim + i] = std::cos(phase);
            out[t * dim + half + i] = std::sin(phase);
        }
}

// ---------------------------------------------------------------------------
// Model (host.rs, config.rs, weights.rs)
// ---------------------------------------------------------------------------

struct Tensor {
    std::vector<float> data;
    std::vector<int64_t> shape;
    int64_t numel() const { return (int64_t)data.size(); }
};

struct Conv {
    const Tensor *w = nullptr, *b = nullptr;
};

struct DConvLayer {
    Conv conv1, conv2;
    const Tensor *n1w, *n1b, *n2w, *n2b, *gamma;
};

struct Layer {  // encoder or decoder
    Conv conv, rewrite;  // conv = conv_tr for decoders
    std::vector<DConvLayer> dconv;
};

struct TLayer {
    bool cross;
    std::vector<float> wq, wk, wv, bq, bk, bv;  // split from in_proj (weights.rs:404-428)
    const Tensor *wo, *bo, *w1, *b1, *w2, *b2;
    const Tensor *n1w, *n1b, *n2w, *n2b, *n3w = nullptr, *n3b = nullptr, *now_, *nob, *g1, *g2;
};

struct Trace {
    dmx_trace_wants_fn wants;
    dmx_trace_record_fn record;
    void *user;
    bool want(const std::string &name) const { return record && (!wants || wants(name.c_str(), user)); }
    void put(const std::string &name, const float *data, std::initializer_list<int64_t> shape) const {
        if (!want(name)) return;
        std::vector<int64_t> s(shape);
        record(name.c_str(), s.data(), (int32_t)s.size(), data, user);
    }
};

}  // namespace

struct oracle_model {
    dmx_config cfg;
    std::map<std::string, Tensor> tensors;
    std::vector<Layer> encoder, tencoder, decoder, tdecoder;  // decoders in execution order
    std::vector<float> freq_emb;                              // (rows, channels) x emb_scale
    int64_t freq_emb_rows = 0;
    const Tensor *up_w, *up_b, *upt_w, *upt_b, *down_w, *down_b, *downt_w, *downt_b;
    const Tensor *norm_in_w, *norm_in_b, *norm_in_t_w, *norm_in_t_b;
    std::vector<TLayer> layers, layers_t;
    int64_t training_length = 0, hop = 0, pre_channels = 0, tch = 0, hidden = 0;

    const Tensor &get(const std::string &name, std::initializer_list<int64_t> shape) {
        auto it = tensors.find(name);
        if (it == tensors.end()) fail("weight `" + name + "` not found in checkpoint");
        std::vector<int64_t> want(shape);
        if (it->second.shape != want) {
            std::string s = "weight `" + name + "` shape mismatch";
            fail(s);
        }
        return it->second;
    }
};

namespace {

// `HtdemucsConfig::validate` (config.rs:239-273).
void validate(const dmx_config &c) {
    if (!c.cac) fail("htdemucs config: cac = false is not supported");
    if (c.nfft != 4096) fail("htdemucs config: nfft != 4096 is not supported");
    if (c.kernel_size != 8 || c.stride != 4) fail("htdemucs config: kernel_size/stride other than 8/4");
    if (c.audio_channels != 2) fail("htdemucs config: audio_channels != 2");
    if (c.sources != 4) fail("htdemucs config: a source count other than 4");
    int64_t freqs = c.nfft / 2;
    for (int i = 0; i < c.depth; ++i) {
        if (freqs > 1 && freqs <= c.kernel_size) fail("htdemucs config: a `last_freq` layer");
        if (freqs > 1) freqs /= c.stride;
    }
}

void dconv_forward(const std::vector<DConvLayer> &layers, float *x, int64_t rows, int64_t channels,
                   int64_t t);

}  // namespace

// ----- model construction (weights.rs:479-578, config.rs:325-444) -----
extern "C" oracle_model *oracle_model_create(const dmx_tensor *weights, size_t n, const dmx_config *cfgp) {
    std::unique_ptr<oracle_model> m(new oracle_model());
    try {
        if (!weights || !cfgp) fail("null argument");
        m->cfg = *cfgp;
        const dmx_config &c = m->cfg;
        validate(c);
        for (size_t i = 0; i < n; ++i) {
            Tensor t;
            int64_t count = 1;
            for (int d = 0; d < weights[i].ndim; ++d) {
                t.shape.push_back(weights[i].shape[d]);
                count *= weights[i].shape[d];
            }
            t.data.assign(weights[i].data, weights[i].data + count);
            m->tensors[weights[i].name] = std::move(t);
        }
        m->training_length = (int64_t)(c.segment * (double)c.samplerate);
        m->hop = c.nfft / 4;
        int64_t depth = c.depth, hidden_div = 8;
        int64_t chin = c.audio_channels, chin_z = chin * 2, chout = c.channels, chout_z = c.channels;
        int64_t freqs = c.nfft / 2;
        struct Spec {
            int64_t chin, chout;
        };
        std::vector<Spec> dec_specs, tdec_specs;
        auto dconv = [&](const std::string &prefix, int64_t ch) {
            std::vector<DConvLayer> out;
            int64_t hid = ch / hidden_div;
            for (int d = 0; d < 2; ++d) {
                std::string at = prefix + ".layers." + std::to_string(d);
                DConvLayer L;
                L.conv1 = {&m->get(at + ".0.weight", {hid, ch, 3}), &m->get(at + ".0.bias", {hid})};
                L.n1w = &m->get(at + ".1.weight", {hid});
                L.n1b = &m->get(at + ".1.bias", {hid});
                L.conv2 = {&m->get(at + ".3.weight", {2 * ch, hid, 1}), &m->get(at + ".3.bias", {2 * ch})};
                L.n2w = &m->get(at + ".4.weight", {2 * ch});
                L.n2b = &m->get(at + ".4.bias", {2 * ch});
                L.gamma = &m->get(at + ".6.scale", {ch});
                out.push_back(L);
            }
            return out;
        };
        for (int64_t i = 0; i < depth; ++i) {
            std::string e = "encoder." + std::to_string(i), te = "tencoder." + std::to_string(i);
            Layer L;
            L.conv = {&m->get(e + ".conv.weight", {chout_z, chin_z, 8, 1}), &m->get(e + ".conv.bias", {chout_z})};
            L.rewrite = {&m->get(e + ".rewrite.weight", {2 * chout_z, chout_z, 1, 1}),
                         &m->get(e + ".rewrite.bias", {2 * chout_z})};
            L.dconv = dconv(e + ".dconv", chout_z);
            m->encoder.push_back(L);
            Layer T;
            T.conv = {&m->get(te + ".conv.weight", {chout, chin, 8}), &m->get(te + ".conv.bias", {chout})};
            T.rewrite = {&m->get(te + ".rewrite.weight", {2 * chout, chout, 1}),
                         &m->get(te + ".rewrite.bias", {2 * chout})};
            T.dconv = dconv(te + ".dconv", chout);
            m->tencoder.push_back(T);
            if (i == 0) {
                chin = (int64_t)c.audio_channels * c.sources;
                chin_z = chin * 2;
            }
            dec_specs.push_back({chout_z, chin_z});
            tdec_specs.push_back({chout, chin});
            if (i == 0) m->freq_emb_rows = freqs / c.stride;
            chin = chout;
            chin_z = chout_z;
            chout *= c.growth;
            chout_z *= c.growth;
            freqs /= c.stride;
        }
        // Decoders in execution order: innermost first (config.rs:434-436),
        // named by construction index depth-1-i (weights.rs:507-527).
        for (int64_t i = depth - 1; i >= 0; --i) {
            std::string d = "decoder." + std::to_string(i), td = "tdecoder." + std::to_string(i);
            Spec s = dec_specs[i], ts = tdec_specs[i];
            int64_t ctx = 1 + 2 * c.context;
            Layer L;
            L.conv = {&m->get(d + ".conv_tr.weight", {s.chin, s.chout, 8, 1}), &m->get(d + ".conv_tr.bias", {s.chout})};
            L.rewrite = {&m->get(d + ".rewrite.weight", {2 * s.chin, s.chin, ctx, ctx}),
                         &m->get(d + ".rewrite.bias", {2 * s.chin})};
            L.dconv = dconv(d + ".dconv", s.chin);
            m->decoder.push_back(L);
            Layer T;
            T.conv = {&m->get(td + ".conv_tr.weight", {ts.chin, ts.chout, 8}), &m->get(td + ".conv_tr.bias", {ts.chout})};
            T.rewrite = {&m->get(td + ".rewrite.weight", {2 * ts.chin, ts.chin, ctx}),
                         &m->get(td + ".rewrite.bias", {2 * ts.chin})};
            T.dconv = dconv(td + ".dconv", ts.chin);
            m->tdecoder.push_back(T);
        }
        m->pre_channels = chin_z;  // bottleneck channels (384)
        m->tch = c.bottom_channels > 0 ? c.bottom_channels : m->pre_channels;
        m->hidden = (int64_t)((double)m->tch * c.t_hidden_scale);
        const Tensor &emb = m->get("freq_emb.embedding.weight", {m->freq_emb_rows, c.channels});
        m->freq_emb.resize(emb.data.size());
        for (size_t i = 0; i < emb.data.size(); ++i) m->freq_emb[i] = emb.data[i] * (float)c.emb_scale;
        int64_t D = m->tch, P = m->pre_channels, H = m->hidden;
        if (c.bottom_channels > 0) {
            m->up_w = &m->get("channel_upsampler.weight", {D, P, 1});
            m->up_b = &m->get("channel_upsampler.bias", {D});
            m->upt_w = &m->get("channel_upsampler_t.weight", {D, P, 1});
            m->upt_b = &m->get("channel_upsampler_t.bias", {D});
            m->down_w = &m->get("channel_downsampler.weight", {P, D, 1});
            m->down_b = &m->get("channel_downsampler.bias", {P});
            m->downt_w = &m->get("channel_downsampler_t.weight", {P, D, 1});
            m->downt_b = &m->get("channel_downsampler_t.bias", {P});
        }
        m->norm_in_w = &m->get("crosstransformer.norm_in.weight", {D});
        m->norm_in_b = &m->get("crosstransformer.norm_in.bias", {D});
        m->norm_in_t_w = &m->get("crosstransformer.norm_in_t.weight", {D});
        m->norm_in_t_b = &m->get("crosstransformer.norm_in_t.bias", {D});
        for (int i = 0; i < c.t_layers; ++i) {
            for (int branch = 0; branch < 2; ++branch) {
                std::string p = std::string(branch ? "crosstransformer.layers_t." : "crosstransformer.layers.") +
                                std::to_string(i);
                TLayer L;
                L.cross = i % 2 == 1;
                std::string a = p + (L.cross ? ".cross_attn" : ".self_attn");
                const Tensor &inw = m->get(a + ".in_proj_weight", {3 * D, D});
                const Tensor &inb = m->get(a + ".in_proj_bias", {3 * D});
                L.wq.assign(inw.data.begin(), inw.data.begin() + D * D);
                L.wk.assign(inw.data.begin() + D * D, inw.data.begin() + 2 * D * D);
                L.wv.assign(inw.data.begin() + 2 * D * D, inw.data.end());
                L.bq.assign(inb.data.begin(), inb.data.begin() + D);
                L.bk.assign(inb.data.begin() + D, inb.data.begin() + 2 * D);
                L.bv.assign(inb.data.begin() + 2 * D, inb.data.end());
                L.wo = &m->get(a + ".out_proj.weight", {D, D});
                L.bo = &m->get(a + ".out_proj.bias", {D});
                L.w1 = &m->get(p + ".linear1.weight", {H, D});
                L.b1 = &m->get(p + ".linear1.bias", {H});
                L.w2 = &m->get(p + ".linear2.weight", {D, H});
                L.b2 = &m->get(p + ".linear2.bias", {D});
                L.n1w = &m->get(p + ".norm1.weight", {D});
                L.n1b = &m->get(p + ".norm1.bias", {D});
                L.n2w = &m->get(p + ".norm2.weight", {D});
                L.n2b = &m->get(p + ".norm2.bias", {D});
                if (L.cross) {
                    L.n3w = &m->get(p + ".norm3.weight", {D});
                    L.n3b = &m->get(p + ".norm3.bias", {D});
                }
                L.now_ = &m->get(p + ".norm_out.weight", {D});
                L.nob = &m->get(p + ".norm_out.bias", {D});
                L.g1 = &m->get(p + ".gamma_1.scale", {D});
                L.g2 = &m->get(p + ".gamma_2.scale", {D});
                (branch ? m->layers_t : m->layers).push_back(std::move(L));
            }
        }
        g_error.clear();
        return m.release();
    } catch (const std::exception &e) {
        g_error = e.what();
        return nullptr;
    }
}

namespace {

// `dconv_forward` (host.rs:985-1059) on (rows, channels, t), in place:
// conv1d k3 (dilation 2^d) -> GN(1) -> GELU -> dconv_tail_into
// (demucs/ops.rs:930-1094): 1x1 -> GN(1) -> GLU -> LayerScale -> +residual.
void dconv_forward(const std::vector<DConvLayer> &layers, float *x, int64_t rows, int64_t channels,
                   int64_t t) {
    for (size_t d = 0; d < layers.size(); ++d) {
        const DConvLayer &L = layers[d];
        int64_t dil = (int64_t)1 << d, hid = L.conv1.w->shape[0];
        std::vector<float> y(rows * hid * t), yn(rows * hid * t);
        conv2d(x, rows, channels, 1, t, L.conv1.w->data.data(), L.conv1.b->data.data(), hid, 1, 3, 1, 1, 0,
               dil, 1, dil, y.data());
        group_norm(y.data(), rows, hid, t, 1, L.n1w->data.data(), L.n1b->data.data(), yn.data());
        gelu_inplace(yn.data(), (int64_t)yn.size());
        int64_t oc = 2 * channels;
#pragma omp parallel for schedule(dynamic) if (!omp_in_parallel())
        for (int64_t r = 0; r < rows; ++r) {
            std::vector<float> z(oc * t);
            sgemm(oc, t, hid, L.conv2.w->data.data(), hid, 1, yn.data() + r * hid * t, t, 1, z.data(), t);
            for (int64_t o = 0; o < oc; ++o) {
                float s = L.conv2.b->data[o];
                if (s != 0.0f)
                    for (int64_t i = 0; i < t; ++i) z[o * t + i] += s;
            }
            Moments mo = moments_f64(z.data(), oc * t);
            float *dst = x + r * channels * t;
            for (int64_t c = 0; c < channels; ++c) {
                float vs = mo.inv * L.n2w->data[c], vsh = L.n2b->data[c] - mo.mean * vs;
                float gs = mo.inv * L.n2w->data[c + channels], gsh = L.n2b->data[c + channels] - mo.mean * gs;
                float ls = L.gamma->data[c];
                for (int64_t i = 0; i < t; ++i) {
                    float value = z[c * t + i] * vs + vsh;
                    float gate = z[(c + channels) * t + i] * gs + gsh;
                    dst[c * t + i] += ls * (value * sigmoid_ref(gate));
                }
            }
        }
    }
}

// (b, c, f, t) <-> (b*f, c, t) (demucs/ops.rs:1517-1581).
void to_rows(const float *x, int64_t b, int64_t c, int64_t f, int64_t t, float *out) {
#pragma omp parallel for schedule(static) if (!omp_in_parallel())
    for (int64_t row = 0; row < b * f; ++row) {
        int64_t bi = row / f, fi = row % f;
        for (int64_t ci = 0; ci < c; ++ci)
            std::memcpy(out + (row * c + ci) * t, x + ((bi * c + ci) * f + fi) * t, t * sizeof(float));
    }
}
void from_rows(const float *x, int64_t b, int64_t c, int64_t f, int64_t t, float *out) {
#pragma omp parallel for schedule(static) if (!omp_in_parallel())
    for (int64_t bc = 0; bc < b * c; ++bc) {
        int64_t bi = bc / c, ci = bc % c;
        for (int64_t fi = 0; fi < f; ++fi)
            std::memcpy(out + (bc * f + fi) * t, x + ((bi * f + fi) * c + ci) * t, t * sizeof(float));
    }
}

std::string idx(const char *base, int64_t i) { return std::string(base) + std::to_string(i); }

// `freq_encoder_forward` (host.rs:577-622): (b, cin, f, t) -> (b, cout, f/4, t).
std::vector<float> freq_encoder(const oracle_model &m, const Layer &L, const std::vector<float> &x,
                                int64_t b, int64_t cin, int64_t f, int64_t t, int64_t &f_out,
                                const Trace &tr, const std::string &name) {
    int64_t cout = L.conv.w->shape[0];
    f_out = (f + 4 - 8) / 4 + 1;
    std::vector<float> y(b * cout * f_out * t);
    conv2d(x.data(), b, cin, f, t, L.conv.w->data.data(), L.conv.b->data.data(), cout, 8, 1, 4, 1, 2, 0,
           1, 1, y.data());
    tr.put(name + ".conv", y.data(), {b, cout, f_out, t});
    gelu_inplace(y.data(), (int64_t)y.size());
    std::vector<float> rows(y.size());
    to_rows(y.data(), b, cout, f_out, t, rows.data());
    dconv_forward(L.dconv, rows.data(), b * f_out, cout, t);
    tr.put(name + ".dconv", rows.data(), {b * f_out, cout, t});
    from_rows(rows.data(), b, cout, f_out, t, y.data());
    std::vector<float> rw(b * 2 * cout * f_out * t), out(b * cout * f_out * t);
    conv2d(y.data(), b, cout, f_out, t, L.rewrite.w->data.data(), L.rewrite.b->data.data(), 2 * cout, 1, 1,
           1, 1, 0, 0, 1, 1, rw.data());
    tr.put(name + ".rewrite", rw.data(), {b, 2 * cout, f_out, t});
    glu(rw.data(), b, 2 * cout, f_out * t, out.data());
    (void)m;
    return out;
}

// `time_encoder_forward` (host.rs:625-678): (b, cin, len) -> (b, cout, ceil(len/4)).
std::vector<float> time_encoder(const Layer &L, const std::vector<float> &x, int64_t b, int64_t cin,
                                int64_t len, int64_t &len_out, const Trace &tr, const std::string &name) {
    int64_t cout = L.conv.w->shape[0];
    int64_t padded = len % 4 ? len + (4 - len % 4) : len;
    std::vector<float> xp;
    const float *src = x.data();
    if (padded != len) {
        xp.assign(b * cin * padded, 0.0f);
        for (int64_t r = 0; r < b * cin; ++r) std::memcpy(xp.data() + r * padded, x.data() + r * len, len * sizeof(float));
        src = xp.data();
    }
    len_out = (padded + 4 - 8) / 4 + 1;
    std::vector<float> y(b * cout * len_out);
    conv2d(src, b, cin, 1, padded, L.conv.w->data.data(), L.conv.b->data.data(), cout, 1, 8, 1, 4, 0, 2, 1,
           1, y.data());
    tr.put(name + ".conv", y.data(), {b, cout, len_out});
    gelu_inplace(y.data(), (int64_t)y.size());
    dconv_forward(L.dconv, y.data(), b, cout, len_out);
    tr.put(name + ".dconv", y.data(), {b, cout, len_out});
    std::vector<float> rw(b * 2 * cout * len_out), out(b * cout * len_out);
    conv2d(y.data(), b, cout, 1, len_out, L.rewrite.w->data.data(), L.rewrite.b->data.data(), 2 * cout, 1, 1,
           1, 1, 0, 0, 1, 1, rw.data());
    tr.put(name + ".rewrite", rw.data(), {b, 2 * cout, len_out});
    glu(rw.data(), b, 2 * cout, len_out, out.data());
    return out;
}

// `freq_decoder_forward` (host.rs:682-759).
std::vector<float> freq_decoder(const Layer &L, const std::vector<float> &x, const std::vector<float> &skip,
                                int64_t b, int64_t cin, int64_t f, int64_t t, bool last, int64_t &f_out,
                                std::vector<float> &pre, const Trace &tr, const std::string &name) {
    std::vector<float> summed(x.size());
    for (size_t i = 0; i < x.size(); ++i) summed[i] = x[i] + skip[i];
    int64_t k = L.rewrite.w->shape[2];
    std::vector<float> rw(b * 2 * cin * f * t), g(b * cin * f * t);
    conv2d(summed.data(), b, cin, f, t, L.rewrite.w->data.data(), L.rewrite.b->data.data(), 2 * cin, k, k, 1,
           1, k / 2, k / 2, 1, 1, rw.data());
    tr.put(name + ".rewrite", rw.data(), {b, 2 * cin, f, t});
    glu(rw.data(), b, 2 * cin, f * t, g.data());
    std::vector<float> rows(g.size());
    to_rows(g.data(), b, cin, f, t, rows.data());
    dconv_forward(L.dconv, rows.data(), b * f, cin, t);
    tr.put(name + ".dconv", rows.data(), {b * f, cin, t});
    pre.resize(g.size());
    from_rows(rows.data(), b, cin, f, t, pre.data());
    int64_t cout = L.conv.w->shape[1];
    int64_t up = (f - 1) * 4 + 8;
    std::vector<float> u(b * cout * up * t);
    conv_transpose2d(pre.data(), b, cin, f, t, L.conv.w->data.data(), L.conv.b->data.data(), cout, 8, 1, 4, 1,
                     u.data());
    tr.put(name + ".conv_tr", u.data(), {b, cout, up, t});
    int64_t pad = 2;
    if (2 * pad > up) fail(name + ": too few bins to crop");
    f_out = up - 2 * pad;
    std::vector<float> z(b * cout * f_out * t);
    for (int64_t bc = 0; bc < b * cout; ++bc)
        std::memcpy(z.data() + bc * f_out * t, u.data() + (bc * up + pad) * t, f_out * t * sizeof(float));
    if (!last) gelu_inplace(z.data(), (int64_t)z.size());
    return z;
}

// `time_decoder_forward` (host.rs:763-827).
std::vector<float> time_decoder(const Layer &L, const std::vector<float> &x, const std::vector<float> &skip,
                                int64_t b, int64_t cin, int64_t len, int64_t length, bool last,
                                std::vector<float> &pre, const Trace &tr, const std::string &name) {
    std::vector<float> summed(x.size());
    for (size_t i = 0; i < x.size(); ++i) summed[i] = x[i] + skip[i];
    int64_t k = L.rewrite.w->shape[2];
    std::vector<float> rw(b * 2 * cin * len);
    pre.resize(b * cin * len);
    conv2d(summed.data(), b, cin, 1, len, L.rewrite.w->data.data(), L.rewrite.b->data.data(), 2 * cin, 1, k, 1,
           1, 0, k / 2, 1, 1, rw.data());
    tr.put(name + ".rewrite", rw.data(), {b, 2 * cin, len});
    glu(rw.data(), b, 2 * cin, len, pre.data());
    dconv_forward(L.dconv, pre.data(), b, cin, len);
    tr.put(name + ".dconv", pre.data(), {b, cin, len});
    int64_t cout = L.conv.w->shape[1];
    int64_t up = (len - 1) * 4 + 8;
    std::vector<float> u(b * cout * up);
    conv_transpose2d(pre.data(), b, cin, 1, len, L.conv.w->data.data(), L.conv.b->data.data(), cout, 1, 8, 1, 4,
                     u.data());
    tr.put(name + ".conv_tr", u.data(), {b, cout, up});
    int64_t pad = 2;
    if (pad + length > up) fail(name + ": transposed convolution produced too few samples");
    std::vector<float> z(b * cout * length);
    for (int64_t bc = 0; bc < b * cout; ++bc)
        std::memcpy(z.data() + bc * length, u.data() + bc * up + pad, length * sizeof(float));
    if (!last) gelu_inplace(z.data(), (int64_t)z.size());
    return z;
}

// `classic_layer_forward` / `cross_layer_forward` (host.rs:1315-1429).
std::vector<float> transformer_layer(const oracle_model &m, const TLayer &L, const std::vector<float> &x,
                                     int64_t n_q, const std::vector<float> *kv, int64_t n_k, int64_t b,
                                     const Trace &tr, const std::string &name) {
    int64_t D = m.tch, H = m.hidden, heads = m.cfg.t_heads;
    std::vector<float> nq(b * n_q * D), attn(b * n_q * D), out(b * n_q * D);
    layer_norm_rows(x.data(), b * n_q, D, L.n1w->data.data(), L.n1b->data.data(), nq.data());
    tr.put(name + ".norm1", nq.data(), {b, n_q, D});
    std::vector<float> q, k, v;
    const bool want_qkv = tr.want(name + ".attn.q");
    if (L.cross) {
        std::vector<float> nk(b * n_k * D);
        layer_norm_rows(kv->data(), b * n_k, D, L.n2w->data.data(), L.n2b->data.data(), nk.data());
        tr.put(name + ".norm2", nk.data(), {b, n_k, D});
        multi_head_attention(nq.data(), nk.data(), b, n_q, n_k, D, heads, L.wq.data(), L.bq.data(), L.wk.data(),
                             L.bk.data(), L.wv.data(), L.bv.data(), L.wo->data.data(), L.bo->data.data(),
                             attn.data(), want_qkv ? &q : nullptr, want_qkv ? &k : nullptr,
                             want_qkv ? &v : nullptr);
    } else {
        n_k = n_q;
        multi_head_attention(nq.data(), nq.data(), b, n_q, n_q, D, heads, L.wq.data(), L.bq.data(), L.wk.data(),
                             L.bk.data(), L.wv.data(), L.bv.data(), L.wo->data.data(), L.bo->data.data(),
                             attn.data(), want_qkv ? &q : nullptr, want_qkv ? &k : nullptr,
                             want_qkv ? &v : nullptr);
    }
    if (want_qkv) {
        tr.put(name + ".attn.q", q.data(), {b * n_q, D});
        tr.put(name + ".attn.k", k.data(), {b * n_k, D});
        tr.put(name + ".attn.v", v.data(), {b * n_k, D});
    }
    tr.put(name + (L.cross ? ".cross_attn#0" : ".self_attn#0"), attn.data(), {b, n_q, D});
    for (int64_t r = 0; r < b * n_q; ++r)
        for (int64_t c = 0; c < D; ++c) out[r * D + c] = x[r * D + c] + attn[r * D + c] * L.g1->data[c];
    std::vector<float> n2(b * n_q * D), h1(b * n_q * H), f2(b * n_q * D);
    if (L.cross) {
        layer_norm_rows(out.data(), b * n_q, D, L.n3w->data.data(), L.n3b->data.data(), n2.data());
        tr.put(name + ".norm3", n2.data(), {b, n_q, D});
    } else {
        layer_norm_rows(out.data(), b * n_q, D, L.n2w->data.data(), L.n2b->data.data(), n2.data());
        tr.put(name + ".norm2", n2.data(), {b, n_q, D});
    }
    // `feed_forward` (host.rs:1432-1457).
    linear(n2.data(), b * n_q, D, L.w1->data.data(), L.b1->data.data(), H, h1.data());
    tr.put(name + ".linear1", h1.data(), {b, n_q, H});
    gelu_inplace(h1.data(), (int64_t)h1.size());
    linear(h1.data(), b * n_q, H, L.w2->data.data(), L.b2->data.data(), D, f2.data());
    tr.put(name + ".linear2", f2.data(), {b, n_q, D});
    for (int64_t r = 0; r < b * n_q; ++r)
        for (int64_t c = 0; c < D; ++c) out[r * D + c] = out[r * D + c] + f2[r * D + c] * L.g2->data[c];
    group_norm_positions(out.data(), b, n_q, D, L.now_->data.data(), L.nob->data.data());
    tr.put(name + ".norm_out", out.data(), {b, n_q, D});
    tr.put(name, out.data(), {b, n_q, D});
    return out;
}

// `transformer_forward` (host.rs:830-946). x (b, D, f, t), xt (b, D, lt).
void transformer_forward(const oracle_model &m, const float *x, const float *xt, int64_t b, int64_t freqs,
                         int64_t frames, int64_t lt, float *x_out, float *xt_out, const Trace &tr) {
    int64_t D = m.tch, lf = freqs * frames;
    std::vector<float> spec(b * lf * D), time(b * lt * D);
    for (int64_t bi = 0; bi < b; ++bi)
        for (int64_t c = 0; c < D; ++c)
            for (int64_t f = 0; f < freqs; ++f)
                for (int64_t t = 0; t < frames; ++t)
                    spec[(bi * lf + t * freqs + f) * D + c] = x[((bi * D + c) * freqs + f) * frames + t];
    for (int64_t bi = 0; bi < b; ++bi)
        for (int64_t c = 0; c < D; ++c)
            for (int64_t t = 0; t < lt; ++t) time[(bi * lt + t) * D + c] = xt[(bi * D + c) * lt + t];
    std::vector<float> pos2d(lf * D), pos1d(lt * D);
    float mp = (float)m.cfg.t_max_period, wpe = (float)m.cfg.t_weight_pos_embed;
    positions_2d(D, freqs, frames, mp, pos2d.data());
    positions_1d(lt, D, mp, pos1d.data());
    std::vector<float> tmp(spec.size());
    layer_norm_rows(spec.data(), b * lf, D, m.norm_in_w->data.data(), m.norm_in_b->data.data(), tmp.data());
    tr.put("crosstransformer.norm_in", tmp.data(), {b, lf, D});
    for (int64_t bi = 0; bi < b; ++bi)
        for (int64_t i = 0; i < lf * D; ++i) spec[bi * lf * D + i] = tmp[bi * lf * D + i] + pos2d[i] * wpe;
    std::vector<float> tmp_t(time.size());
    layer_norm_rows(time.data(), b * lt, D, m.norm_in_t_w->data.data(), m.norm_in_t_b->data.data(), tmp_t.data());
    tr.put("crosstransformer.norm_in_t", tmp_t.data(), {b, lt, D});
    for (int64_t bi = 0; bi < b; ++bi)
        for (int64_t i = 0; i < lt * D; ++i) time[bi * lt * D + i] = tmp_t[bi * lt * D + i] + pos1d[i] * wpe;
    tr.put("crosstransformer.in#0", spec.data(), {b, lf, D});
    tr.put("crosstransformer.in#1", time.data(), {b, lt, D});
    for (int i = 0; i < m.cfg.t_layers; ++i) {
        const TLayer &L = m.layers[i], &LT = m.layers_t[i];
        std::string n = idx("crosstransformer.layers.", i), nt = idx("crosstransformer.layers_t.", i);
        if (L.cross) {
            std::vector<float> old_spec = spec;
            spec = transformer_layer(m, L, spec, lf, &time, lt, b, tr, n);
            time = transformer_layer(m, LT, time, lt, &old_spec, lf, b, tr, nt);
        } else {
            spec = transformer_layer(m, L, spec, lf, nullptr, 0, b, tr, n);
            time = transformer_layer(m, LT, time, lt, nullptr, 0, b, tr, nt);
        }
    }
    for (int64_t bi = 0; bi < b; ++bi)
        for (int64_t c = 0; c < D; ++c)
            for (int64_t f = 0; f < freqs; ++f)
                for (int64_t t = 0; t < frames; ++t)
                    x_out[((bi * D + c) * freqs + f) * frames + t] = spec[(bi * lf + t * freqs + f) * D + c];
    for (int64_t bi = 0; bi < b; ++bi)
        for (int64_t c = 0; c < D; ++c)
            for (int64_t t = 0; t < lt; ++t) xt_out[(bi * D + c) * lt + t] = time[(bi * lt + t) * D + c];
}

// 1x1 channel map over positions of (b, cin, positions) (host.rs:951-974 and the
// freq-branch permute/linear/permute at host.rs:320-337): out = W x + bias.
void channel_mix(const float *x, int64_t b, int64_t cin, int64_t positions, const Tensor &w, const Tensor &bias,
                 float *out) {
    int64_t cout = w.shape[0];
    for (int64_t bi = 0; bi < b; ++bi) {
        float *dst = out + bi * cout * positions;
        sgemm(cout, positions, cin, w.data.data(), cin, 1, x + bi * cin * positions, positions, 1, dst, positions);
        for (int64_t o = 0; o < cout; ++o)
            for (int64_t p = 0; p < positions; ++p) dst[o * positions + p] += bias.data[o];
    }
}

// `Htdemucs::forward` (host.rs:202-520).
void forward(const oracle_model &m, const float *mix_in, int64_t batch, int64_t channels, int64_t length,
             float *out, const Trace &tr) {
    const dmx_config &c = m.cfg;
    if (channels != c.audio_channels) fail("expected 2 audio channels");
    int64_t L = m.training_length;
    if (length > L) fail("input is longer than the model segment; chunk the audio before calling forward");
    std::vector<float> padded(batch * channels * L, 0.0f);
    for (int64_t r = 0; r < batch * channels; ++r)
        std::memcpy(padded.data() + r * L, mix_in + r * length, length * sizeof(float));
    tr.put("mix.in", padded.data(), {batch, channels, L});
    int64_t nfft = c.nfft, hop = m.hop, le = (L + hop - 1) / hop, fr = nfft / 2;
    int64_t zc = 2 * channels;
    std::vector<float> x(batch * zc * fr * le);
    spec_cac(padded.data(), batch, channels, L, nfft, x.data());
    tr.put("_spec", x.data(), {batch, zc, fr, le});
    tr.put("_magnitude", x.data(), {batch, zc, fr, le});
    // `normalise` (host.rs:523-543) and the affine of host.rs:250-261.
    std::vector<float> mean(batch), stdv(batch), mean_t(batch), std_t(batch);
    int64_t plane = zc * fr * le, wplane = channels * L;
    for (int64_t bi = 0; bi < batch; ++bi) {
        mean[bi] = mean_f64(x.data() + bi * plane, plane);
        stdv[bi] = std_unbiased(x.data() + bi * plane, plane);
        mean_t[bi] = mean_f64(padded.data() + bi * wplane, wplane);
        std_t[bi] = std_unbiased(padded.data() + bi * wplane, wplane);
    }
    std::vector<float> xt = padded;
    for (int64_t bi = 0; bi < batch; ++bi) {
        float off = mean[bi], sc = 1.0f / (1e-5f + stdv[bi]);
        for (int64_t i = 0; i < plane; ++i) x[bi * plane + i] = (x[bi * plane + i] - off) * sc;
        float offt = mean_t[bi], sct = 1.0f / (1e-5f + std_t[bi]);
        for (int64_t i = 0; i < wplane; ++i) xt[bi * wplane + i] = (xt[bi * wplane + i] - offt) * sct;
    }
    tr.put("x_normalized", x.data(), {batch, zc, fr, le});
    tr.put("xt_normalized", xt.data(), {batch, channels, L});

    int64_t depth = c.depth;
    std::vector<std::vector<float>> saved, saved_t;
    std::vector<int64_t> lengths, lengths_t, cs, cts, fs;
    int64_t cin = zc, f = fr, tcin = channels, tlen = L;
    for (int64_t i = 0; i < depth; ++i) {
        lengths.push_back(le);
        lengths_t.push_back(tlen);
        int64_t tlen_out;
        std::string tn = idx("tencoder.", i), n = idx("encoder.", i);
        xt = time_encoder(m.tencoder[i], xt, batch, tcin, tlen, tlen_out, tr, tn);
        tcin = m.tencoder[i].conv.w->shape[0];
        tlen = tlen_out;
        tr.put(tn, xt.data(), {batch, tcin, tlen});
        saved_t.push_back(xt);
        int64_t f_out;
        x = freq_encoder(m, m.encoder[i], x, batch, cin, f, le, f_out, tr, n);
        cin = m.encoder[i].conv.w->shape[0];
        f = f_out;
        tr.put(n, x.data(), {batch, cin, f, le});
        if (i == 0 && c.freq_emb > 0.0) {
            // `add_frequency_embedding` (host.rs:546-574).
            if (f != m.freq_emb_rows || cin != c.channels) fail("frequency embedding shape mismatch");
            float scale = (float)c.freq_emb;
            for (int64_t bi = 0; bi < batch; ++bi)
                for (int64_t ch = 0; ch < cin; ++ch)
                    for (int64_t fi = 0; fi < f; ++fi) {
                        float value = scale * m.freq_emb[fi * c.channels + ch];
                        float *run = x.data() + ((bi * cin + ch) * f + fi) * le;
                        for (int64_t t = 0; t < le; ++t) run[t] += value;
                    }
            tr.put("encoder.0.post_emb", x.data(), {batch, cin, f, le});
        }
        saved.push_back(x);
    }
    int64_t D = m.tch, P = m.pre_channels;
    if (c.bottom_channels > 0) {
        std::vector<float> up(batch * D * f * le), upt(batch * D * tlen);
        channel_mix(x.data(), batch, P, f * le, *m.up_w, *m.up_b, up.data());
        channel_mix(xt.data(), batch, P, tlen, *m.upt_w, *m.upt_b, upt.data());
        x.swap(up);
        xt.swap(upt);
    }
    tr.put("channel_upsampler", x.data(), {batch, D, f * le});
    tr.put("channel_upsampler_t", xt.data(), {batch, D, tlen});
    tr.put("crosstransformer#0", x.data(), {batch, D, f, le});
    tr.put("crosstransformer#1", xt.data(), {batch, D, tlen});
    std::vector<float> xo(x.size()), xto(xt.size());
    transformer_forward(m, x.data(), xt.data(), batch, f, le, tlen, xo.data(), xto.data(), tr);
    x.swap(xo);
    xt.swap(xto);
    if (c.bottom_channels > 0) {
        std::vector<float> dn(batch * P * f * le), dnt(batch * P * tlen);
        channel_mix(x.data(), batch, D, f * le, *m.down_w, *m.down_b, dn.data());
        channel_mix(xt.data(), batch, D, tlen, *m.downt_w, *m.downt_b, dnt.data());
        x.swap(dn);
        xt.swap(dnt);
    }
    tr.put("channel_downsampler", x.data(), {batch, P, f * le});
    tr.put("channel_downsampler_t", xt.data(), {batch, P, tlen});
    cin = P;
    tcin = P;
    for (int64_t i = 0; i < depth; ++i) {
        bool last = i == depth - 1;
        std::vector<float> skip = std::move(saved.back());
        saved.pop_back();
        lengths.pop_back();
        std::vector<float> pre;
        int64_t f_out;
        std::string n = idx("decoder.", i), tn = idx("tdecoder.", i);
        std::vector<float> z = freq_decoder(m.decoder[i], x, skip, batch, cin, f, le, last, f_out, pre, tr, n);
        int64_t cout = m.decoder[i].conv.w->shape[1];
        tr.put(n + "#0", z.data(), {batch, cout, f_out, le});
        tr.put(n + "#1", pre.data(), {batch, cin, f, le});
        x.swap(z);
        cin = cout;
        f = f_out;
        std::vector<float> skip_t = std::move(saved_t.back());
        saved_t.pop_back();
        int64_t length_t = lengths_t.back();
        lengths_t.pop_back();
        std::vector<float> pre_t;
        std::vector<float> zt = time_decoder(m.tdecoder[i], xt, skip_t, batch, tcin, tlen, length_t, last, pre_t, tr, tn);
        int64_t tcout = m.tdecoder[i].conv.w->shape[1];
        tr.put(tn + "#0", zt.data(), {batch, tcout, length_t});
        tr.put(tn + "#1", pre_t.data(), {batch, tcin, tlen});
        xt.swap(zt);
        tcin = tcout;
        tlen = length_t;
    }
    int64_t S = c.sources;
    if (cin != S * 4) fail("the frequency branch produced the wrong channel count");
    // Denormalise (host.rs:466-469): affine(x, -m/s, s) = (x + m/s) * s.
    for (int64_t bi = 0; bi < batch; ++bi) {
        float sc = stdv[bi], off = -mean[bi] / sc;
        int64_t n = S * 4 * fr * le;
        for (int64_t i = 0; i < n; ++i) x[bi * n + i] = (x[bi * n + i] - off) * sc;
    }
    tr.put("_mask.in", x.data(), {batch, S, 4, fr, le});
    std::vector<float> wave(batch * S * channels * L);
    ispec_cac(x.data(), batch, S, fr, le, nfft, L, wave.data());
    tr.put("_ispec.out", wave.data(), {batch, S, channels, L});
    tr.put("time_branch_out", xt.data(), {batch, S, channels, L});
    for (int64_t bi = 0; bi < batch; ++bi) {
        float sc = std_t[bi], off = -mean_t[bi] / sc;
        int64_t n = S * channels * L;
        for (int64_t i = 0; i < n; ++i) xt[bi * n + i] = (xt[bi * n + i] - off) * sc;
    }
    for (int64_t bi = 0; bi < batch; ++bi)
        for (int64_t r = 0; r < S * channels; ++r)
            for (int64_t t = 0; t < length; ++t) {
                int64_t src = (bi * S * channels + r) * L + t;
                out[(bi * S * channels + r) * length + t] = xt[src] + wave[src];
            }
    tr.put("model_out", out, {batch, S, channels, length});
}

// `transition_weight` (pipeline.rs:117-131).
std::vector<float> transition_weight(int64_t n, double power) {
    std::vector<float> w;
    int64_t half = n / 2;
    for (int64_t i = 1; i <= half; ++i) w.push_back((float)i);
    for (int64_t i = n - half; i >= 1; --i) w.push_back((float)i);
    float mx = 1.0f;
    for (float v : w) mx = std::max(mx, v);
    for (float &v : w) v = std::pow(v / mx, (float)power);
    return w;
}

// `ShiftRng` (pipeline.rs:136-151).
struct ShiftRng {
    uint64_t s;
    explicit ShiftRng(uint64_t seed) : s(seed * 6364136223846793005ULL + 1ULL) {}
    int64_t randint(int64_t max) {
        s = s * 6364136223846793005ULL + 1442695040888963407ULL;
        return (int64_t)((s >> 33) % (uint64_t)(max + 1));
    }
};

// One `stream_split_pass` (streaming.rs:296-400) over a normalised mix
// (batch, channels, mix_len), with the optional shift view
// (mix.rs:587-640). Returns (batch, sources, channels, view_len) OLA output
// (already divided by the summed weights), accumulated in segment order so
// it is bit-identical to the O(segment) ring.
std::vector<float> split_pass(const float *mix, int64_t batch, int64_t channels, int64_t mix_len,
                              int64_t seg, double overlap, double power, int64_t shift_offset,
                              int64_t max_shift, int64_t group, int64_t sources,
                              const std::function<void(const std::vector<float> &, int64_t, std::vector<float> &)> &fwd,
                              int64_t &view_len) {
    int64_t stride = (int64_t)((1.0 - overlap) * (double)seg);
    if (stride == 0) fail("overlap leaves a zero stride");
    std::vector<float> weight = transition_weight(seg, power);
    view_len = max_shift > 0 ? mix_len + max_shift - shift_offset : mix_len;
    std::vector<float> acc(batch * sources * channels * std::max<int64_t>(view_len, 0), 0.0f);
    std::vector<float> sum_w(std::max<int64_t>(view_len, 0), 0.0f);
    int64_t offset = 0;
    while (offset < view_len) {
        std::vector<std::pair<int64_t, int64_t>> spans;
        int64_t cursor = offset;
        while ((int64_t)spans.size() < group && cursor < view_len) {
            spans.push_back({cursor, std::min(view_len - cursor, seg)});
            cursor += stride;
        }
        int64_t g = (int64_t)spans.size();
        std::vector<float> batched(g * batch * channels * seg, 0.0f);
        for (int64_t slot = 0; slot < g; ++slot) {
            int64_t start = spans[slot].first - (seg - spans[slot].second) / 2;
            for (int64_t b = 0; b < batch; ++b)
                for (int64_t ch = 0; ch < channels; ++ch)
                    for (int64_t i = 0; i < seg; ++i) {
                        int64_t vi = start + i;
                        float sample = 0.0f;
                        if (vi >= 0 && vi < view_len) {
                            int64_t mi = max_shift > 0 ? shift_offset + vi - max_shift : vi;
                            if (mi >= 0 && mi < mix_len) sample = mix[(b * channels + ch) * mix_len + mi];
                        }
                        batched[((slot * batch + b) * channels + ch) * seg + i] = sample;
                    }
        }
        std::vector<float> out_g(g * batch * sources * channels * seg);
        fwd(batched, g * batch, out_g);
        for (int64_t slot = 0; slot < g; ++slot) {
            int64_t s0 = spans[slot].first, cl = spans[slot].second, trim = (seg - cl) / 2;
            for (int64_t b = 0; b < batch; ++b)
                for (int64_t r = 0; r < sources * channels; ++r) {
                    const float *src = out_g.data() + ((slot * batch + b) * sources * channels + r) * seg + trim;
                    float *dst = acc.data() + (b * sources * channels + r) * view_len + s0;
                    for (int64_t t = 0; t < cl; ++t) dst[t] += weight[t] * src[t];
                }
            for (int64_t t = 0; t < cl; ++t) sum_w[s0 + t] += weight[t];
        }
        offset = cursor;
    }
    for (int64_t t = 0; t < view_len; ++t)
        if (sum_w[t] <= 0.0f) fail("overlap-add left a sample with no weight");
    for (int64_t r = 0; r < batch * sources * channels; ++r)
        for (int64_t t = 0; t < view_len; ++t) acc[r * view_len + t] /= sum_w[t];
    return acc;
}

}  // namespace

// ============================ C API ==========================================
extern "C" {

const char *oracle_last_error(void) { return g_error.c_str(); }
void oracle_set_threads(int threads) {
    if (threads > 0) omp_set_num_threads(threads);
}
int oracle_get_threads(void) { return omp_get_max_threads(); }

void oracle_sgemm(int64_t m, int64_t n, int64_t k, const float *a, int64_t a_rs, int64_t a_cs, const float *b,
                  int64_t b_rs, int64_t b_cs, float *c, int64_t ldc) {
    sgemm(m, n, k, a, a_rs, a_cs, b, b_rs, b_cs, c, ldc);
}

int oracle_conv2d(const float *x, int64_t batch, int64_t ic, int64_t h, int64_t w, const float *weight,
                  const float *bias, int64_t oc, int64_t kh, int64_t kw, int64_t sh, int64_t sw, int64_t ph,
                  int64_t pw, int64_t dh, int64_t dw, float *out) {
    return guarded([&] { conv2d(x, batch, ic, h, w, weight, bias, oc, kh, kw, sh, sw, ph, pw, dh, dw, out); });
}

int oracle_conv_transpose2d(const float *x, int64_t batch, int64_t ic, int64_t h, int64_t w, const float *weight,
                            const float *bias, int64_t oc, int64_t kh, int64_t kw, int64_t sh, int64_t sw,
                            float *out) {
    return guarded([&] { conv_transpose2d(x, batch, ic, h, w, weight, bias, oc, kh, kw, sh, sw, out); });
}

int oracle_group_norm(const float *x, int64_t batch, int64_t channels, int64_t inner, int64_t groups,
                      const float *weight, const float *bias, float *out) {
    return guarded([&] { group_norm(x, batch, channels, inner, groups, weight, bias, out); });
}

int oracle_group_norm_glu(const float *x, int64_t batch, int64_t channels, int64_t inner, int64_t groups,
                          const float *weight, const float *bias, float *out) {
    return guarded([&] { group_norm_glu(x, batch, channels, inner, groups, weight, bias, out); });
}

int oracle_layer_norm_rows(const float *x, int64_t rows, int64_t dim, const float *weight, const float *bias,
                           float *out) {
    return guarded([&] { layer_norm_rows(x, rows, dim, weight, bias, out); });
}

int oracle_glu(const float *x, int64_t batch, int64_t channels, int64_t inner, float *out) {
    return guarded([&] { glu(x, batch, channels, inner, out); });
}

void oracle_gelu(const float *x, int64_t n, float *out) {
    for (int64_t i = 0; i < n; ++i) out[i] = gelu(x[i]);
}
float oracle_gelu_scalar(float x) { return gelu(x); }
float oracle_mean(const float *x, int64_t n) { return mean_f64(x, n); }
float oracle_std_unbiased(const float *x, int64_t n) { return std_unbiased(x, n); }

int oracle_attention_head(const float *q, const float *k, const float *v, int64_t n_q, int64_t n_k,
                          int64_t d_head, float scale, float *out) {
    return guarded([&] { attention_head(q, d_head, k, d_head, v, d_head, n_q, n_k, d_head, scale, out, d_head); });
}

int oracle_multi_head_attention(const float *query, const float *key, int64_t batch, int64_t n_q, int64_t n_k,
                                int64_t dim, int64_t heads, const float *wq, const float *bq, const float *wk,
                                const float *bk, const float *wv, const float *bv, const float *wo,
                                const float *bo, float *out) {
    return guarded([&] {
        multi_head_attention(query, key, batch, n_q, n_k, dim, heads, wq, bq, wk, bk, wv, bv, wo, bo, out);
    });
}

int oracle_dconv(const float *x, int64_t rows, int64_t channels, int64_t t, const dmx_tensor *w, size_t n,
                 const char *prefix, float *out) {
    return guarded([&] {
        std::map<std::string, Tensor> tensors;
        for (size_t i = 0; i < n; ++i) {
            Tensor tt;
            int64_t count = 1;
            for (int d = 0; d < w[i].ndim; ++d) {
                tt.shape.push_back(w[i].shape[d]);
                count *= w[i].shape[d];
            }
            tt.data.assign(w[i].data, w[i].data + count);
            tensors[w[i].name] = std::move(tt);
        }
        auto get = [&](const std::string &name) -> const Tensor * {
            auto it = tensors.find(name);
            if (it == tensors.end()) fail("weight `" + name + "` not found");
            return &it->second;
        };
        std::vector<DConvLayer> layers;
        for (int d = 0; d < 2; ++d) {
            std::string at = std::string(prefix) + ".layers." + std::to_string(d);
            DConvLayer L;
            L.conv1 = {get(at + ".0.weight"), get(at + ".0.bias")};
            L.n1w = get(at + ".1.weight");
            L.n1b = get(at + ".1.bias");
            L.conv2 = {get(at + ".3.weight"), get(at + ".3.bias")};
            L.n2w = get(at + ".4.weight");
            L.n2b = get(at + ".4.bias");
            L.gamma = get(at + ".6.scale");
            layers.push_back(L);
        }
        std::memcpy(out, x, rows * channels * t * sizeof(float));
        dconv_forward(layers, out, rows, channels, t);
    });
}

void oracle_hann_window(int64_t n, float *out) {
    std::vector<float> w = hann(n);
    std::copy(w.begin(), w.end(), out);
}

void oracle_fft(const float *re, const float *im, int64_t n, int inverse, double *out_re, double *out_im) {
    std::vector<double> r(re, re + n), i(n, 0.0);
    if (im) i.assign(im, im + n);
    dft(r, i, inverse ? +1 : -1);
    std::copy(r.begin(), r.end(), out_re);
    std::copy(i.begin(), i.end(), out_im);
}

int oracle_stft(const float *x, int64_t batch, int64_t samples, int64_t n_fft, int64_t hop, int normalized,
                float *out_re, float *out_im, int64_t *frames_out) {
    return guarded([&] {
        int64_t frames = 1 + samples / hop;
        if (frames_out) *frames_out = frames;
        if (out_re) stft(x, batch, samples, n_fft, hop, normalized != 0, out_re, out_im);
    });
}

int oracle_istft(const float *re, const float *im, int64_t batch, int64_t bins, int64_t frames, int64_t n_fft,
                 int64_t hop, int normalized, int64_t length, float *out, int64_t *out_len) {
    return guarded([&] {
        int64_t n = istft(re, im, batch, bins, frames, n_fft, hop, normalized != 0, length, nullptr);
        if (out_len) *out_len = n;
        if (out) istft(re, im, batch, bins, frames, n_fft, hop, normalized != 0, length, out);
    });
}

int oracle_pad1d_reflect(const float *x, int64_t length, int64_t left, int64_t right, float *out) {
    return guarded([&] {
        std::vector<float> v = pad1d_reflect(x, length, left, right);
        std::copy(v.begin(), v.end(), out);
    });
}

int oracle_spec_cac(const float *mix, int64_t batch, int64_t channels, int64_t length, int64_t nfft, float *out) {
    return guarded([&] { spec_cac(mix, batch, channels, length, nfft, out); });
}

int oracle_ispec_cac(const float *x, int64_t batch, int64_t sources, int64_t bins, int64_t le, int64_t nfft,
                     int64_t length, float *out) {
    return guarded([&] { ispec_cac(x, batch, sources, bins, le, nfft, length, out); });
}

void oracle_positions_2d(int64_t dim, int64_t height, int64_t width, float max_period, float *out) {
    positions_2d(dim, height, width, max_period, out);
}
void oracle_positions_1d(int64_t length, int64_t dim, float max_period, float *out) {
    positions_1d(length, dim, max_period, out);
}
void oracle_transition_weight(int64_t segment_length, double power, float *out) {
    std::vector<float> w = transition_weight(segment_length, power);
    std::copy(w.begin(), w.end(), out);
}
void oracle_shift_rng(uint64_t seed, int64_t max, int64_t count, int64_t *out) {
    ShiftRng rng(seed);
    for (int64_t i = 0; i < count; ++i) out[i] = rng.randint(max);
}

void oracle_scan_norm(const float *wav, int64_t batch, int64_t channels, int64_t length, float *mean,
                      float *std_out) {
    double count = (double)(batch * length), sum = 0.0, sum_sq = 0.0;
    for (int64_t b = 0; b < batch; ++b)
        for (int64_t t = 0; t < length; ++t) {
            double acc = 0.0;
            for (int64_t c = 0; c < channels; ++c) acc += (double)wav[(b * channels + c) * length + t];
            double r = acc / (double)channels;
            sum += r;
            sum_sq += r * r;
        }
    double m = sum / count;
    double var = count > 1.0 ? (sum_sq - sum * sum / count) / (count - 1.0) : 0.0;
    *mean = (float)m;
    *std_out = (float)std::sqrt(std::max(var, 0.0)) + 1e-8f;
}

void oracle_model_destroy(oracle_model *model) { delete model; }
int64_t oracle_model_training_length(const oracle_model *model) { return model ? model->training_length : 0; }

int oracle_forward(oracle_model *model, const float *mix, int64_t batch, int64_t channels, int64_t length,
                   float *out, dmx_trace_wants_fn wants, dmx_trace_record_fn record, void *user) {
    return guarded([&] {
        if (!model || !mix || !out) fail("null argument");
        forward(*model, mix, batch, channels, length, out, Trace{wants, record, user});
    });
}

int oracle_transformer_forward(oracle_model *model, const float *x, const float *xt, int64_t batch,
                               int64_t freqs, int64_t frames, int64_t time_len, float *x_out, float *xt_out,
                               dmx_trace_wants_fn wants, dmx_trace_record_fn record, void *user) {
    return guarded([&] {
        if (!model) fail("null model");
        transformer_forward(*model, x, xt, batch, freqs, frames, time_len, x_out, xt_out,
                            Trace{wants, record, user});
    });
}

int oracle_split_pass(const float *mix, int64_t batch, int64_t channels, int64_t length, int64_t segment_length,
                      double overlap, double transition_power, int64_t shift_offset, int64_t max_shift,
                      int32_t batch_chunks, int32_t sources, oracle_forward_fn fwd, void *user, float *out) {
    return guarded([&] {
        int64_t view_len = 0;
        auto f = [&](const std::vector<float> &padded, int64_t b, std::vector<float> &o) {
            if (fwd(padded.data(), b, channels, segment_length, o.data(), user) != 0) fail("forward callback failed");
        };
        std::vector<float> acc = split_pass(mix, batch, channels, length, segment_length, overlap, transition_power,
                                            shift_offset, max_shift, std::max(1, batch_chunks), sources, f, view_len);
        std::copy(acc.begin(), acc.end(), out);
    });
}

// `Demucs::run_channels` -> `run_mix` -> `separate_streaming_normalized_mix`
// (api.rs:474-545, 697-785) with `separate_forwarding_emit` (pipeline.rs:380-515)
// and the bag's `BagCombineForward` (api.rs:319-371).
int oracle_separate(oracle_model *const *nets, const float *bag_weights, int32_t n_nets, const uint8_t *stems_wanted,
                    const float *left, const float *right, int64_t samples, int32_t sample_rate,
                    const dmx_separate_options *opts, oracle_forward_fn fwd, void *fwd_user, int32_t sources_arg,
                    float *stems_out) {
    return guarded([&] {
        if (!left || !right || !opts || !stems_out) fail("null argument");
        if (!fwd && (n_nets < 1 || !nets)) fail("no network");
        const int64_t channels = 2;
        int64_t sources = fwd ? sources_arg : nets[0]->cfg.sources;
        int32_t sr = fwd ? sample_rate : nets[0]->cfg.samplerate;
        if (sample_rate != sr) fail("audio sample rate does not match the model");
        double seg_s = opts->segment > 0 ? opts->segment : (fwd ? 0.0 : nets[0]->cfg.segment);
        int64_t seg = (int64_t)((double)sr * seg_s);
        if (fwd && opts->segment <= 0) fail("a callback forward needs an explicit segment");
        std::vector<float> mix(channels * samples);
        std::memcpy(mix.data(), left, samples * sizeof(float));
        std::memcpy(mix.data() + samples, right, samples * sizeof(float));
        float gm, gs;
        oracle_scan_norm(mix.data(), 1, channels, samples, &gm, &gs);
        for (float &v : mix) v = (v - gm) / gs;
        std::vector<bool> requested(sources, true);
        if (stems_wanted)
            for (int64_t s = 0; s < sources; ++s) requested[s] = stems_wanted[s] != 0;
        // One group's forward: single network, bag combine, or the callback.
        auto group_forward = [&](const std::vector<float> &padded, int64_t b, std::vector<float> &out) {
            if (fwd) {
                if (fwd(padded.data(), b, channels, seg, out.data(), fwd_user) != 0) fail("forward callback failed");
                return;
            }
            if (n_nets == 1 && !bag_weights) {
                forward(*nets[0], padded.data(), b, channels, seg, out.data(), Trace{nullptr, nullptr, nullptr});
                return;
            }
            std::fill(out.begin(), out.end(), 0.0f);
            std::vector<float> totals(sources, 0.0f), one(out.size());
            for (int32_t n = 0; n < n_nets; ++n) {
                const float *wrow = bag_weights + n * sources;
                bool needed = false;
                for (int64_t s = 0; s < sources; ++s) needed |= wrow[s] != 0.0f && requested[s];
                if (!needed) continue;
                forward(*nets[n], padded.data(), b, channels, seg, one.data(), Trace{nullptr, nullptr, nullptr});
                for (int64_t s = 0; s < sources; ++s) {
                    if (wrow[s] == 0.0f || !requested[s]) continue;
                    for (int64_t bi = 0; bi < b; ++bi)
                        for (int64_t i = 0; i < channels * seg; ++i) {
                            int64_t at = ((bi * sources + s) * channels) * seg + i;
                            out[at] += one[at] * wrow[s];
                        }
                    totals[s] += wrow[s];
                }
            }
            for (int64_t s = 0; s < sources; ++s) {
                if (!requested[s]) continue;
                if (totals[s] == 0.0f) fail("no network covers stem index " + std::to_string(s));
                for (int64_t bi = 0; bi < b; ++bi)
                    for (int64_t i = 0; i < channels * seg; ++i) out[((bi * sources + s) * channels) * seg + i] /= totals[s];
            }
        };
        int64_t max_shift = (int64_t)(0.5 * (double)sr);
        ShiftRng rng(0x5eed1234ULL);
        int32_t shifts = opts->shifts;
        int64_t group = std::max(1, opts->batch_chunks);
        std::vector<float> result(sources * channels * samples, 0.0f);
        if (shifts == 0) {
            int64_t vl;
            result = split_pass(mix.data(), 1, channels, samples, seg, opts->overlap, opts->transition_power, 0, 0, group,
                                sources, group_forward, vl);
        } else {
            float scale = 1.0f / (float)shifts;
            for (int32_t pass = 0; pass < shifts; ++pass) {
                int64_t offset = rng.randint(max_shift), trim = max_shift - offset, vl;
                std::vector<float> acc = split_pass(mix.data(), 1, channels, samples, seg, opts->overlap,
                                                    opts->transition_power, offset, max_shift, group, sources,
                                                    group_forward, vl);
                for (int64_t r = 0; r < sources * channels; ++r)
                    for (int64_t t = 0; t < samples; ++t) {
                        int64_t tv = t + trim;
                        if (tv < vl) {
                            if (shifts == 1)
                                result[r * samples + t] = acc[r * vl + tv] * scale;
                            else
                                result[r * samples + t] += acc[r * vl + tv];
                        }
                    }
            }
            if (shifts > 1)
                for (float &v : result) v *= scale;
        }
        for (int64_t s = 0; s < sources; ++s) {
            if (!requested[s]) continue;
            for (int64_t i = 0; i < channels * samples; ++i)
                stems_out[s * channels * samples + i] = result[s * channels * samples + i] * gs + gm;
        }
    });
}

}  // extern "C"
