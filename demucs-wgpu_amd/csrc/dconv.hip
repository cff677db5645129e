// dconv.hip — the DConv residual layer for narrow branches (hidden = C/8 <= 12),
// as three direct VALU passes with one thread per time position.
//
// Semantics: `dconv_forward` + `dconv_tail_into`
// (crates/demucs-core/src/demucs/host.rs:985-1059, demucs/ops.rs:930-1094):
//   y = conv1d_k3_dil(x) + b1;      GN(1, H) over (H, T) per row; GELU
//   z = W2 . gelu(GN(y)) + b2;      GN(1, 2C) over (2C, T) per row
//   x += gamma * (GN(z)[c] * sigmoid(GN(z)[C + c]))
// With H <= 12 a 32-row MFMA tile would be >60% padding, and each pass is
// bound by one sweep over x; these kernels do the useful FMAs only. The rows
// are the (b, f) rows of a (B, C, F, T) tensor, addressed in place.
//   pass 1: conv1 -> y (rows, H, T), GN1 statistics
//   pass 2: GN1+GELU (on load) -> W2 -> GN2 statistics only
//   pass 3: GN1+GELU -> W2 -> GN2 -> GLU -> LayerScale -> += into x
// Recomputing W2 in pass 3 (2C*H FMAs per position) is cheaper than writing
// and re-reading the 2C-channel intermediate.
#include "common.h"
#include "ops.h"

namespace dmx {
namespace {

constexpr int DC_THREADS = 256;
constexpr int DC_MAX_C = 96;

__device__ __forceinline__ const float *row_base(const float *x, int z, int C, int F, int T) {
    int b = z / F, f = z - b * F;
    return x + ((int64_t)b * C * F + f) * T;
}

template <int H>
__global__ __launch_bounds__(DC_THREADS) void dconv_conv1_kernel(const float *__restrict__ x, int C, int F, int T,
                                                                 int dil, const float *__restrict__ w1,
                                                                 const float *__restrict__ b1, float *__restrict__ y,
                                                                 double *__restrict__ stats) {
    __shared__ float ws[H * DC_MAX_C * 3];
    const int z = blockIdx.y;
    for (int i = threadIdx.x; i < H * C * 3; i += DC_THREADS) ws[i] = w1[i];
    __syncthreads();
    const int t = blockIdx.x * DC_THREADS + threadIdx.x;
    const bool ok = t < T;
    const float *xr = row_base(x, z, C, F, T);
    const int64_t cs = (int64_t)F * T;
    float acc[H];
#pragma unroll
    for (int h = 0; h < H; ++h) acc[h] = 0.0f;
    if (ok) {
        const bool l_ok = t - dil >= 0, r_ok = t + dil < T;
        for (int c = 0; c < C; ++c) {
            const float *xc = xr + c * cs;
            float x0 = l_ok ? xc[t - dil] : 0.0f, x1 = xc[t], x2 = r_ok ? xc[t + dil] : 0.0f;
#pragma unroll
            for (int h = 0; h < H; ++h) {
                const float *w = ws + (h * C + c) * 3;
                acc[h] += w[0] * x0 + w[1] * x1 + w[2] * x2;
            }
        }
    }
    double s = 0.0, q = 0.0;
    if (ok) {
        float *yr = y + (int64_t)z * H * T + t;
#pragma unroll
        for (int h = 0; h < H; ++h) {
            float v = acc[h] + b1[h];
            yr[(int64_t)h * T] = v;
            s += v;
            q += (double)v * v;
        }
    }
    block_moments_atomic(s, q, stats + 2 * z);
}

// GN1 + GELU of this position's H conv1 outputs.
template <int H>
__device__ __forceinline__ void load_hidden(const float *y, int z, int T, int t, const double *stats1,
                                            const float *n1w, const float *n1b, float g[H]) {
    float mean, inv;
    gn_stats(stats1 + 2 * z, (double)H * T, mean, inv);
    const float *yr = y + (int64_t)z * H * T + t;
#pragma unroll
    for (int h = 0; h < H; ++h) {
        float scale = inv * n1w[h];
        float shift = n1b[h] - mean * scale;
        g[h] = gelu(yr[(int64_t)h * T] * scale + shift);
    }
}

template <int H>
__global__ __launch_bounds__(DC_THREADS) void dconv_conv2_stats_kernel(const float *__restrict__ y, int C, int T,
                                                                       const double *__restrict__ stats1,
                                                                       const float *__restrict__ n1w,
                                                                       const float *__restrict__ n1b,
                                                                       const float *__restrict__ w2,
                                                                       const float *__restrict__ b2,
                                                                       double *__restrict__ stats2) {
    __shared__ float ws[2 * DC_MAX_C * H];
    __shared__ float bs[2 * DC_MAX_C];
    const int z = blockIdx.y;
    for (int i = threadIdx.x; i < 2 * C * H; i += DC_THREADS) ws[i] = w2[i];
    for (int i = threadIdx.x; i < 2 * C; i += DC_THREADS) bs[i] = b2[i];
    __syncthreads();
    const int t = blockIdx.x * DC_THREADS + threadIdx.x;
    double s = 0.0, q = 0.0;
    if (t < T) {
        float g[H];
        load_hidden<H>(y, z, T, t, stats1, n1w, n1b, g);
        for (int o = 0; o < 2 * C; ++o) {
            float v = 0.0f;
#pragma unroll
            for (int h = 0; h < H; ++h) v += ws[o * H + h] * g[h];
            v += bs[o];
            s += v;
            q += (double)v * v;
        }
    }
    block_moments_atomic(s, q, stats2 + 2 * z);
}

template <int H>
__global__ __launch_bounds__(DC_THREADS) void dconv_apply_kernel(float *__restrict__ x, const float *__restrict__ y,
                                                                 int C, int F, int T, const double *__restrict__ stats1,
                                                                 const float *__restrict__ n1w,
                                                                 const float *__restrict__ n1b,
                                                                 const float *__restrict__ w2,
                                                                 const float *__restrict__ b2,
                                                                 const double *__restrict__ stats2,
                                                                 const float *__restrict__ n2w,
                                                                 const float *__restrict__ n2b,
                                                                 const float *__restrict__ gamma) {
    __shared__ float ws[2 * DC_MAX_C * H];
    __shared__ float bs[2 * DC_MAX_C], sc[2 * DC_MAX_C], sh[2 * DC_MAX_C], gm[DC_MAX_C];
    const int z = blockIdx.y;
    float mean2, inv2;
    gn_stats(stats2 + 2 * z, 2.0 * C * (double)T, mean2, inv2);
    for (int i = threadIdx.x; i < 2 * C * H; i += DC_THREADS) ws[i] = w2[i];
    for (int i = threadIdx.x; i < 2 * C; i += DC_THREADS) {
        bs[i] = b2[i];
        float scale = inv2 * n2w[i];
        sc[i] = scale;
        sh[i] = n2b[i] - mean2 * scale;
    }
    for (int i = threadIdx.x; i < C; i += DC_THREADS) gm[i] = gamma[i];
    __syncthreads();
    const int t = blockIdx.x * DC_THREADS + threadIdx.x;
    if (t >= T) return;
    float g[H];
    load_hidden<H>(y, z, T, t, stats1, n1w, n1b, g);
    float *xr = const_cast<float *>(row_base(x, z, C, F, T)) + t;
    const int64_t cs = (int64_t)F * T;
    for (int c = 0; c < C; ++c) {
        float v = 0.0f, u = 0.0f;
#pragma unroll
        for (int h = 0; h < H; ++h) {
            v += ws[c * H + h] * g[h];
            u += ws[(C + c) * H + h] * g[h];
        }
        float value = (v + bs[c]) * sc[c] + sh[c];
        float gate = (u + bs[C + c]) * sc[C + c] + sh[C + c];
        xr[c * cs] += gm[c] * (value * sigmoid(gate));
    }
}

template <int H>
void launch_all(hipStream_t s, float *x, int B, int C, int F, int T, int dil, const float *w1, const float *b1,
                const float *n1w, const float *n1b, const float *w2, const float *b2, const float *n2w,
                const float *n2b, const float *gamma, float *hbuf, double *stats) {
    const int rows = B * F;
    double *st1 = stats, *st2 = stats + 2 * rows;
    dim3 grid((unsigned)ceil_div(T, DC_THREADS), (unsigned)rows);
    hipLaunchKernelGGL(dconv_conv1_kernel<H>, grid, dim3(DC_THREADS), 0, s, x, C, F, T, dil, w1, b1, hbuf, st1);
    DMX_LAUNCH_CHECK();
    hipLaunchKernelGGL(dconv_conv2_stats_kernel<H>, grid, dim3(DC_THREADS), 0, s, hbuf, C, T, st1, n1w, n1b, w2, b2,
                       st2);
    DMX_LAUNCH_CHECK();
    hipLaunchKernelGGL(dconv_apply_kernel<H>, grid, dim3(DC_THREADS), 0, s, x, hbuf, C, F, T, st1, n1w, n1b, w2, b2,
                       st2, n2w, n2b, gamma);
    DMX_LAUNCH_CHECK();
}

}  // namespace

bool dconv_layer_narrow(hipStream_t s, float *x, int B, int C, int F, int T, int dil, const float *w1,
                        const float *b1, int H, const float *n1w, const float *n1b, const float *w2, const float *b2,
                        const float *n2w, const float *n2b, const float *gamma, float *hbuf, double *stats) {
    if (C > DC_MAX_C || B * F > 65535) return false;
    if (H == 6 && C == 48)
        launch_all<6>(s, x, B, C, F, T, dil, w1, b1, n1w, n1b, w2, b2, n2w, n2b, gamma, hbuf, stats);
    else if (H == 12 && C == 96)
        launch_all<12>(s, x, B, C, F, T, dil, w1, b1, n1w, n1b, w2, b2, n2w, n2b, gamma, hbuf, stats);
    else
        return false;
    return true;
}

}  // namespace dmx
