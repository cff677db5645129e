// dconv.hip — the DConv residual layer for narrow branches (C = 48 or 96,
// hidden H = C/8 = 6 or 12).
//
// Semantics: `dconv_forward` + `dconv_tail_into`
// (crates/demucs-core/src/demucs/host.rs:985-1059, demucs/ops.rs:930-1094):
//   y = conv1d_k3_dil(x) + b1;      GN(1, H) over (H, T) per row; GELU
//   z = W2 . gelu(GN(y)) + b2;      GN(1, 2C) over (2C, T) per row
//   x += gamma * (GN(z)[c] * sigmoid(GN(z)[C + c]))
// The rows are the (b, f) rows of a (B, C, F, T) tensor, addressed in place.
//
// With H <= 12 a matrix-core tile would be mostly padding, so the two
// contractions run on the VALU, one thread per position, 64 positions per
// wave. Every weight and per-row coefficient is indexed uniformly across the
// wave, so it is a scalar load and an SGPR operand: one VALU instruction per
// FMA, no LDS traffic. Launches:
//   0. W1 (H, C, 3) -> (C, 3, H), so each channel's 3H weights are contiguous.
//   1. y = conv1(x) + b1, plus partial moments of y per 64 positions.
//   2. per row: GN1 moments in f64 -> GN1 as an affine (scale, shift) per h.
//   3. g = GELU(GN1(y)); per wave (up to 256 positions) the sums
//      S_h = sum_t g_h and the Gram matrix G_hh' = sum_t g_h g_h' (h <= h').
//   4. per row: those partials in f64, and GN2's moments from them, since
//      z_o = W2[o] . g + b2[o] gives
//        sum_t z_o   = W2[o] . S + T b2[o]
//        sum_t z_o^2 = W2[o] G W2[o]^T + 2 b2[o] (W2[o] . S) + T b2[o]^2;
//      GN2 (with b2 folded in) as an affine per channel o.
//   5. z = W2 g, GN2, GLU, LayerScale, += into x.
// x crosses HBM three times (two reads, one write); the 2C-channel z is never
// stored and never formed for its statistics. Row reductions go through
// partials, not same-address atomics (those serialise on the long time rows).
// Loads read a clamped index unconditionally and are multiplied by a 0/1 mask
// (a select lets the compiler turn each load into a branch); the data is
// finite, so the product is exactly the zero padding.
#include <type_traits>

#include "common.h"
#include "ops.h"

namespace dmx {
namespace {

constexpr int DC_THREADS = 256;  // 4 waves, one work item each
constexpr int C1_POS = 64;       // positions per conv1 / apply work item
constexpr int GR_ITER = 4;       // 64-position chunks per Gram work item
constexpr float DC_LOG2E = 1.4426950408889634f;

template <int H>
constexpr int gram_terms() {
    return H + H * (H + 1) / 2;
}

// Scratch layout inside `hbuf` (floats).
struct NarrowScratch {
    float *y, *part1, *aff1, *part, *aff2, *w1t;
};
template <int C, int H>
NarrowScratch carve(float *hbuf, int rows, int T) {
    NarrowScratch s;
    const int64_t items64 = (int64_t)rows * ceil_div(T, C1_POS);
    const int64_t items_g = (int64_t)rows * ceil_div(T, C1_POS * GR_ITER);
    s.y = hbuf;
    s.part1 = s.y + (int64_t)rows * H * T;
    s.aff1 = s.part1 + 2 * items64;
    s.part = s.aff1 + (int64_t)rows * H * 2;
    s.aff2 = s.part + items_g * gram_terms<H>();
    s.w1t = s.aff2 + (int64_t)rows * 2 * C * 2;
    return s;
}

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

__device__ __forceinline__ float *row_ptr(float *x, int z, int C, int F, int T) {
    int b = z / F, f = z - b * F;
    return x + ((int64_t)b * C * F + f) * T;
}

__device__ __forceinline__ float fast_sigmoid(float v) {
    return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-v * DC_LOG2E));
}

__global__ void dconv_w1_transpose_kernel(const float *__restrict__ w1, int C, int H, float *__restrict__ w1t) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;  // i = (h * C + c) * 3 + k
    if (i >= H * C * 3) return;
    const int h = i / (C * 3), ck = i - h * C * 3;
    w1t[ck * H + h] = w1[i];
}

// 1. y = conv1(x) + b1; per-item (sum, sum of squares) of y.
template <int C, int H>
__global__ __launch_bounds__(DC_THREADS) void dconv_conv1_kernel(const float *__restrict__ x, int F, int T, int dil,
                                                                 int items_per_row, int n_items,
                                                                 const float *__restrict__ w1t,
                                                                 const float *__restrict__ b1, float *__restrict__ y,
                                                                 float *__restrict__ part1) {
    const int lane = threadIdx.x & 63;
    const int item = uniform(blockIdx.x * 4 + (threadIdx.x >> 6));
    if (item >= n_items) return;
    const int z = uniform(item / items_per_row);
    const int t = (item - z * items_per_row) * C1_POS + lane;
    const float *xr = row_ptr(const_cast<float *>(x), z, C, F, T);
    const int64_t cs = (int64_t)F * T;
    const int tl = t - dil, tr = t + dil;
    const int il = min(max(tl, 0), T - 1), ic = min(t, T - 1), ir = min(tr, T - 1);
    const float ml = tl >= 0 && tl < T ? 1.0f : 0.0f, mc = t < T ? 1.0f : 0.0f, mr = tr < T ? 1.0f : 0.0f;
    float acc[H];
#pragma unroll
    for (int h = 0; h < H; ++h) acc[h] = b1[h];
#pragma unroll 4
    for (int c = 0; c < C; ++c) {
        const float *xc = xr + c * cs;
        const float x0 = xc[il] * ml, x1 = xc[ic] * mc, x2 = xc[ir] * mr;
        const float *w = w1t + c * 3 * H;
#pragma unroll
        for (int h = 0; h < H; ++h) acc[h] = fmaf(w[h], x0, fmaf(w[H + h], x1, fmaf(w[2 * H + h], x2, acc[h])));
    }
    float fs = 0.0f, fq = 0.0f;
    if (t < T) {
        float *yr = y + (int64_t)z * H * T + t;
#pragma unroll
        for (int h = 0; h < H; ++h) {
            yr[(int64_t)h * T] = acc[h];
            fs += acc[h];
            fq += acc[h] * acc[h];
        }
    }
    fs = wave_sum(fs);
    fq = wave_sum(fq);
    if (lane == 0) {
        part1[2 * item] = fs;
        part1[2 * item + 1] = fq;
    }
}

// One block sums the NS-term partials of row z in f64 into `out` (LDS): the
// block's threads split into 256 / NS groups, thread (j, i) sums term i over
// items j, j + groups, ..., then one thread per term adds the groups.
template <int NS>
__device__ void sum_row_partials(const float *part, int items_per_row, int z, double *out) {
    static_assert(NS <= DC_THREADS, "one thread per term at least");
    constexpr int GROUPS = DC_THREADS / NS;
    __shared__ double red[GROUPS * NS];
    const int i = threadIdx.x % NS, j = threadIdx.x / NS;
    const float *p = part + (int64_t)z * items_per_row * NS + i;
    if (j < GROUPS) {
        double a = 0.0;
        for (int it = j; it < items_per_row; it += GROUPS) a += (double)p[(int64_t)it * NS];
        red[j * NS + i] = a;
    }
    __syncthreads();
    if (threadIdx.x < NS) {
        double a = 0.0;
        for (int g = 0; g < GROUPS; ++g) a += red[g * NS + threadIdx.x];
        out[threadIdx.x] = a;
    }
    __syncthreads();
}

// 2. GN1 of row z as (scale, shift) per hidden channel.
__global__ __launch_bounds__(DC_THREADS) void dconv_gn1_kernel(const float *__restrict__ part1, int items_per_row,
                                                               int H, int T, const float *__restrict__ n1w,
                                                               const float *__restrict__ n1b,
                                                               float *__restrict__ aff1) {
    __shared__ double sums[2];
    const int z = blockIdx.x;
    sum_row_partials<2>(part1, items_per_row, z, sums);
    if (threadIdx.x < H) {
        float mean, inv;
        gn_stats(sums, (double)H * T, mean, inv);
        const int h = threadIdx.x;
        const float scale = inv * n1w[h];
        aff1[(z * H + h) * 2] = scale;
        aff1[(z * H + h) * 2 + 1] = n1b[h] - mean * scale;
    }
}

// GN1 + GELU of the H hidden channels at position t (clamped; masked by m).
template <int H>
__device__ __forceinline__ void hidden(const float *y, int z, int T, int t, float m, const float *aff1, float g[H]) {
    const float *yr = y + (int64_t)z * H * T + min(t, T - 1);
    const float *a = aff1 + z * H * 2;
#pragma unroll
    for (int h = 0; h < H; ++h) g[h] = gelu(yr[(int64_t)h * T] * a[2 * h] + a[2 * h + 1]) * m;
}

// 3. Per wave (GR_ITER chunks of 64 positions): S_h and the upper triangle of
// G, accumulated per lane, then wave-reduced.
template <int H>
__global__ __launch_bounds__(DC_THREADS) void dconv_gram_kernel(const float *__restrict__ y, int T, int items_per_row,
                                                                int n_items, const float *__restrict__ aff1,
                                                                float *__restrict__ part) {
    constexpr int NS = gram_terms<H>();
    const int lane = threadIdx.x & 63;
    const int item = uniform(blockIdx.x * 4 + (threadIdx.x >> 6));
    if (item >= n_items) return;
    const int z = uniform(item / items_per_row);
    const int t_begin = (item - z * items_per_row) * (C1_POS * GR_ITER);
    float acc[NS];
#pragma unroll
    for (int i = 0; i < NS; ++i) acc[i] = 0.0f;
    for (int c = 0; c < GR_ITER; ++c) {
        if (t_begin + c * C1_POS >= T) break;  // uniform
        const int t = t_begin + c * C1_POS + lane;
        float g[H];
        hidden<H>(y, z, T, t, t < T ? 1.0f : 0.0f, aff1, g);
        int i = 0;
#pragma unroll
        for (int h = 0; h < H; ++h, ++i) acc[i] += g[h];
#pragma unroll
        for (int h = 0; h < H; ++h)
#pragma unroll
            for (int h2 = h; h2 < H; ++h2, ++i) acc[i] = fmaf(g[h], g[h2], acc[i]);
    }
    float *out = part + (int64_t)item * NS;
#pragma unroll
    for (int i = 0; i < NS; ++i) {
        const float v = wave_sum(acc[i]);
        if (lane == 0) out[i] = v;
    }
}

// 4. One block per row: S and G in f64, GN2's moments, GN2 as (scale, shift)
// per channel o with b2 folded into the shift.
template <int C, int H>
__global__ __launch_bounds__(DC_THREADS) void dconv_gn2_kernel(const float *__restrict__ part, int items_per_row,
                                                               int T, const float *__restrict__ w2,
                                                               const float *__restrict__ b2,
                                                               const float *__restrict__ n2w,
                                                               const float *__restrict__ n2b,
                                                               float *__restrict__ aff2) {
    constexpr int NS = gram_terms<H>();
    __shared__ double sg[NS];
    __shared__ double red[2][DC_THREADS / 64];
    __shared__ double mom[2];
    const int z = blockIdx.x;
    sum_row_partials<NS>(part, items_per_row, z, sg);
    auto gram = [&](int h, int h2) -> double {  // G[h][h2] from the stored upper triangle
        if (h > h2) {
            const int t = h;
            h = h2;
            h2 = t;
        }
        return sg[H + h * H - h * (h - 1) / 2 + (h2 - h)];
    };
    double sz = 0.0, sz2 = 0.0;
    for (int o = threadIdx.x; o < 2 * C; o += DC_THREADS) {
        const float *w = w2 + (int64_t)o * H;
        double ws = 0.0, quad = 0.0;
        for (int h = 0; h < H; ++h) {
            ws += (double)w[h] * sg[h];
            double inner = 0.0;
            for (int h2 = 0; h2 < H; ++h2) inner += (double)w[h2] * gram(h, h2);
            quad += (double)w[h] * inner;
        }
        const double b = b2[o];
        sz += ws + (double)T * b;
        sz2 += quad + 2.0 * b * ws + (double)T * b * b;
    }
    sz = wave_sum_d(sz);
    sz2 = wave_sum_d(sz2);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) {
        red[0][wave] = sz;
        red[1][wave] = sz2;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        double a = 0.0, b = 0.0;
        for (int w = 0; w < DC_THREADS / 64; ++w) {
            a += red[0][w];
            b += red[1][w];
        }
        mom[0] = a;
        mom[1] = b;
    }
    __syncthreads();
    float mean, inv;
    gn_stats(mom, 2.0 * C * (double)T, mean, inv);
    for (int o = threadIdx.x; o < 2 * C; o += DC_THREADS) {
        const float scale = inv * n2w[o];
        aff2[(z * 2 * C + o) * 2] = scale;
        aff2[(z * 2 * C + o) * 2 + 1] = n2b[o] + (b2[o] - mean) * scale;
    }
}

// 5. z = W2 g per position, GN2, GLU, LayerScale, += into x.
template <int C, int H>
__global__ __launch_bounds__(DC_THREADS) void dconv_apply_kernel(float *__restrict__ x, const float *__restrict__ y,
                                                                 int F, int T, int items_per_row, int n_items,
                                                                 const float *__restrict__ aff1,
                                                                 const float *__restrict__ w2,
                                                                 const float *__restrict__ aff2,
                                                                 const float *__restrict__ gamma) {
    const int lane = threadIdx.x & 63;
    const int item = uniform(blockIdx.x * 4 + (threadIdx.x >> 6));
    if (item >= n_items) return;
    const int z = uniform(item / items_per_row);
    const int t = (item - z * items_per_row) * C1_POS + lane;
    float g[H];
    hidden<H>(y, z, T, t, 1.0f, aff1, g);
    if (t >= T) return;
    float *xr = row_ptr(x, z, C, F, T) + t;
    const int64_t cs = (int64_t)F * T;
    const float *a2 = aff2 + z * 2 * C * 2;
#pragma unroll 4
    for (int c = 0; c < C; ++c) {
        const float *wv = w2 + c * H, *wg = w2 + (C + c) * H;
        float v = 0.0f, u = 0.0f;
#pragma unroll
        for (int h = 0; h < H; ++h) {
            v = fmaf(wv[h], g[h], v);
            u = fmaf(wg[h], g[h], u);
        }
        const float value = fmaf(v, a2[2 * c], a2[2 * c + 1]);
        const float gate = fmaf(u, a2[2 * (C + c)], a2[2 * (C + c) + 1]);
        xr[c * cs] = fmaf(gamma[c], value * fast_sigmoid(gate), xr[c * cs]);
    }
}

template <int C, int H>
void launch_all(hipStream_t s, float *x, int B, int F, int T, int dil, const float *w1, const float *w1_t,
                const float *b1, const float *n1w, const float *n1b, const float *w2, const float *b2,
                const float *n2w, const float *n2b, const float *gamma, float *hbuf) {
    const int rows = B * F;
    const NarrowScratch sc = carve<C, H>(hbuf, rows, T);
    const int per_row64 = ceil_div(T, C1_POS), per_row_g = ceil_div(T, C1_POS * GR_ITER);
    const int items64 = rows * per_row64, items_g = rows * per_row_g;
    if (!w1_t) {
        hipLaunchKernelGGL(dconv_w1_transpose_kernel, dim3((unsigned)ceil_div(H * C * 3, 256)), dim3(256), 0, s, w1, C,
                           H, sc.w1t);
        DMX_LAUNCH_CHECK();
        w1_t = sc.w1t;
    }
    hipLaunchKernelGGL((dconv_conv1_kernel<C, H>), dim3((unsigned)ceil_div(items64, 4)), dim3(DC_THREADS), 0, s, x, F,
                       T, dil, per_row64, items64, w1_t, b1, sc.y, sc.part1);
    DMX_LAUNCH_CHECK();
    hipLaunchKernelGGL(dconv_gn1_kernel, dim3((unsigned)rows), dim3(DC_THREADS), 0, s, sc.part1, per_row64, H, T, n1w,
                       n1b, sc.aff1);
    DMX_LAUNCH_CHECK();
    hipLaunchKernelGGL(dconv_gram_kernel<H>, dim3((unsigned)ceil_div(items_g, 4)), dim3(DC_THREADS), 0, s, sc.y, T,
                       per_row_g, items_g, sc.aff1, sc.part);
    DMX_LAUNCH_CHECK();
    hipLaunchKernelGGL((dconv_gn2_kernel<C, H>), dim3((unsigned)rows), dim3(DC_THREADS), 0, s, sc.part, per_row_g, T,
                       w2, b2, n2w, n2b, sc.aff2);
    DMX_LAUNCH_CHECK();
    hipLaunchKernelGGL((dconv_apply_kernel<C, H>), dim3((unsigned)ceil_div(items64, 4)), dim3(DC_THREADS), 0, s, x,
                       sc.y, F, T, per_row64, items64, sc.aff1, w2, sc.aff2, gamma);
    DMX_LAUNCH_CHECK();
}

// ---------------------------------------------------------------------------
// Both DConv layers of a short row in one launch (`dconv_forward`'s loop over
// depth, host.rs:984-1059): one workgroup per (b, f) row holds the row, C x T,
// in LDS with a zero halo of RW_PAD positions on each side, runs layer 0
// (dilation 1) and layer 1 (dilation 2) on it, and writes it back once — x
// crosses HBM once each way for the two layers, and nothing else does (the
// hidden activations, their moments and the GN affines stay in LDS).
//
// Threads: RW_GROUPS groups of RW_WAVES waves, one position per lane (T <=
// RW_TMAX). In conv1 group j computes hidden channels [j H/G, (j+1) H/G) of
// its position, in the apply channels [j C/G, (j+1) C/G); the group index is
// uniform per wave, so every weight is a scalar load. The moments follow the
// narrow path above: GN1 from per-thread sums, GN2 from S_h and the Gram
// matrix of the hidden activations, both reduced in f64.
constexpr int RW_WAVES = 6;                 // waves per group
constexpr int RW_TMAX = 64 * RW_WAVES;      // longest row
constexpr int RW_GROUPS = 2;
constexpr int RW_THREADS = 64 * RW_WAVES * RW_GROUPS;
constexpr int RW_PAD = 4;                   // >= the largest dilation (2); keeps rows 16-byte aligned
constexpr int RW_LDS_BYTES = 160 * 1024;    // gfx950 LDS per workgroup

struct RowLayers {  // kernel argument: both layers' weights
    DConvRowLayer l[2];
};

// LDS carve-up, in bytes from the start of the dynamic allocation; every
// section starts 16-byte aligned.
template <int C, int H>
struct RowLds {
    static constexpr int NS = gram_terms<H>();
    // Weights in LDS (WL): each layer's W2 (2C, H) in its own section and W1
    // as [group][c][tap][H / G] (W1P floats per (group, c)) over the hidden
    // rows, which conv1 does not use; without WL they are scalar loads.
    static constexpr bool WL = C >= 96;
    static constexpr int W1P = ((3 * H / RW_GROUPS + 3) / 4) * 4;
    static constexpr int red = 0;                                  // float [RW_THREADS]
    static constexpr int sg = red + RW_THREADS * 4;                // double [NS]
    static constexpr int wsum = sg + ((NS * 8 + 15) / 16) * 16;    // double [2 passes][waves][2]
    static constexpr int coef = wsum + 2 * (RW_THREADS / 64) * 2 * 8;  // float4 [C]
    static constexpr int w2s = coef + C * 16;                      // float [2C][H] (WL)
    static constexpr int xs = w2s + (WL ? 2 * C * H * 4 : 0);      // float [C][T + 2 PAD]
    __host__ __device__ static int gs(int T) { return xs + C * (T + 2 * RW_PAD) * 4; }  // float [H][T | 1]
    __host__ __device__ static int bytes(int T) {
        const int hidden = H * (T | 1) * 4, w1 = WL ? RW_GROUPS * C * W1P * 4 : 0;
        return gs(T) + (hidden > w1 ? hidden : w1);
    }
};

// Sum over the wave with DPP moves (no LDS round trips): pairs, quads, half
// rows and rows by quad_perm / mirrors, then rows 0+1 and 2+3 by row_bcast15
// and the whole wave by row_bcast31 into lane 63, read from there.
__device__ __forceinline__ float wave_sum_dpp(float v) {
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xb1, 0xf, 0xf, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4e, 0xf, 0xf, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xf, 0xf, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xf, 0xf, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x142, 0xa, 0xf, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x143, 0xc, 0xf, false));
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Sum (a, b) over the workgroup: f32 within each wave (a wave's terms are a
// few products each), f64 across waves. `buf` holds 2 doubles per wave and
// must not be reused before the next barrier.
__device__ __forceinline__ void block_sum2(double &a, double &b, double *buf) {
    a = wave_sum_dpp((float)a);
    b = wave_sum_dpp((float)b);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) {
        buf[2 * wave] = a;
        buf[2 * wave + 1] = b;
    }
    __syncthreads();
    a = 0.0;
    b = 0.0;
#pragma unroll
    for (int w = 0; w < RW_THREADS / 64; ++w) {
        a += buf[2 * w];
        b += buf[2 * w + 1];
    }
}

// Row (C, T) between HBM (channel stride cs) and LDS (channel stride S,
// data from RW_PAD): thread -> (channel offset, V positions), channels
// advancing by RW_THREADS / (T / V); RW_BATCH channels' loads are issued
// before the first LDS write (indices clamped, writes guarded).
constexpr int RW_BATCH = 8;
template <int C, int V, bool IN>
__device__ __forceinline__ void row_copy(float *xr, int64_t cs, float *xs, int S, int T) {
    using vec = typename std::conditional<V == 4, float4, float>::type;
    const int TV = T / V, cstep = RW_THREADS / TV, c0 = threadIdx.x / TV, tv = (threadIdx.x - c0 * TV) * V;
    if (c0 >= cstep) return;
    for (int c = c0; c < C; c += RW_BATCH * cstep) {
        vec v[RW_BATCH];
#pragma unroll
        for (int k = 0; k < RW_BATCH; ++k) {
            const int cc = min(c + k * cstep, C - 1);
            v[k] = IN ? *reinterpret_cast<const vec *>(xr + cc * cs + tv)
                      : *reinterpret_cast<const vec *>(xs + cc * S + RW_PAD + tv);
        }
#pragma unroll
        for (int k = 0; k < RW_BATCH; ++k) {
            const int cc = c + k * cstep;
            if (cc < C) {
                if (IN)
                    *reinterpret_cast<vec *>(xs + cc * S + RW_PAD + tv) = v[k];
                else
                    *reinterpret_cast<vec *>(xr + cc * cs + tv) = v[k];
            }
        }
    }
}

template <int C, int H>
__device__ __forceinline__ void row_layer(char *lds, int T, int dil, const DConvRowLayer &L) {
    using Lay = RowLds<C, H>;
    constexpr int NS = Lay::NS, HG = H / RW_GROUPS, CG = C / RW_GROUPS;
    float *red = reinterpret_cast<float *>(lds + Lay::red);
    double *sg = reinterpret_cast<double *>(lds + Lay::sg);
    double *wsum = reinterpret_cast<double *>(lds + Lay::wsum);
    float4 *coef = reinterpret_cast<float4 *>(lds + Lay::coef);
    float *xs = reinterpret_cast<float *>(lds + Lay::xs);
    float *gs = reinterpret_cast<float *>(lds + Lay::gs(T));
    const int S = T + 2 * RW_PAD, TG = T | 1;  // odd hidden-row stride: the Gram pass reads rows at one t
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = uniform(tid >> 6);
    const int grp = uniform(wave / RW_WAVES);
    const int t = (wave - grp * RW_WAVES) * 64 + lane;
    const bool live = t < T;
    const int tc = min(t, T - 1) + RW_PAD;  // lanes past the row read its last position
    float *w2s = reinterpret_cast<float *>(lds + Lay::w2s);
    constexpr int W1P = Lay::W1P;

    if constexpr (Lay::WL) {  // this layer's weights into LDS (the previous layer is done with both regions)
        for (int i = tid; i < RW_GROUPS * C * 3 * HG; i += RW_THREADS) {
            const int gc = i / (3 * HG), r = i - gc * (3 * HG), g = gc / C, c = gc - g * C;
            const int k = r / HG, j = r - k * HG;
            gs[gc * W1P + r] = L.w1_t[(c * 3 + k) * H + g * HG + j];
        }
        for (int i = tid; i < 2 * C * H / 4; i += RW_THREADS)
            reinterpret_cast<float4 *>(w2s)[i] = reinterpret_cast<const float4 *>(L.w2)[i];
        __syncthreads();
    }

    // conv1 (k = 3, dilation dil) for hidden channels [grp HG, grp HG + HG).
    float acc[HG];
#pragma unroll
    for (int j = 0; j < HG; ++j) acc[j] = L.b1[grp * HG + j];
    if constexpr (Lay::WL) {
        const float *xc = xs + tc;
        const float4 *wq = reinterpret_cast<const float4 *>(gs + grp * C * W1P);
#pragma unroll 2
        for (int c = 0; c < C; ++c, xc += S, wq += W1P / 4) {
            const float x0 = xc[-dil], x1 = xc[0], x2 = xc[dil];
            float wc[W1P];
#pragma unroll
            for (int i = 0; i < W1P / 4; ++i) {
                const float4 v = wq[i];
                wc[4 * i] = v.x;
                wc[4 * i + 1] = v.y;
                wc[4 * i + 2] = v.z;
                wc[4 * i + 3] = v.w;
            }
#pragma unroll
            for (int j = 0; j < HG; ++j)
                acc[j] = fmaf(wc[j], x0, fmaf(wc[HG + j], x1, fmaf(wc[2 * HG + j], x2, acc[j])));
        }
    } else {
        const float *w = L.w1_t + grp * HG;
        const float *xc = xs + tc;
#pragma unroll 4
        for (int c = 0; c < C; ++c, xc += S) {
            const float x0 = xc[-dil], x1 = xc[0], x2 = xc[dil];
            const float *wc = w + c * 3 * H;
#pragma unroll
            for (int j = 0; j < HG; ++j)
                acc[j] = fmaf(wc[j], x0, fmaf(wc[H + j], x1, fmaf(wc[2 * H + j], x2, acc[j])));
        }
    }
    // GN1 over (H, T), then GELU, into gs.
    {
        double s = 0.0, q = 0.0;
        if (live) {
            float fs = 0.0f, fq = 0.0f;
#pragma unroll
            for (int j = 0; j < HG; ++j) {
                fs += acc[j];
                fq = fmaf(acc[j], acc[j], fq);
            }
            s = fs;
            q = fq;
        }
        block_sum2(s, q, wsum);
        const double m = s / ((double)H * T);
        const float mean = (float)m, inv = 1.0f / (float)sqrt(fmax(q / ((double)H * T) - m * m, 0.0) + 1e-5);
        if (live) {
#pragma unroll
            for (int j = 0; j < HG; ++j) {
                const int h = grp * HG + j;
                const float sc = inv * L.n1w[h];
                gs[h * TG + t] = gelu(fmaf(acc[j], sc, L.n1b[h] - mean * sc));
            }
        }
    }
    __syncthreads();
    // S_h and the upper triangle of G_hh' = sum_t g_h g_h': thread -> (term,
    // chunk of positions); chunk partials in f32, their sum in f64.
    {
        constexpr int J = RW_THREADS / NS;
        const int i = tid % NS, j = tid / NS;
        float part = 0.0f;
        if (j < J) {
            int ha = i, hb = i;
            if (i >= H) {  // pair term: walk the triangle rows
                int k = i - H;
                ha = 0;
                while (k >= H - ha) {
                    k -= H - ha;
                    ++ha;
                }
                hb = ha + k;
            }
            const bool sum_term = i < H;
            const int chunk = (T + J - 1) / J;
            const int t0 = j * chunk, t1 = min(T, t0 + chunk);
            const float *ga = gs + ha * TG, *gb = gs + hb * TG;
            for (int u = t0; u < t1; ++u) part = fmaf(ga[u], sum_term ? 1.0f : gb[u], part);
        }
        red[tid] = part;
        __syncthreads();
        if (tid < NS) {
            double a = 0.0;
            for (int jj = 0; jj < J; ++jj) a += (double)red[jj * NS + tid];
            sg[tid] = a;
        }
        __syncthreads();
    }
    // GN2 moments of z_o = W2[o] . g + b2[o] over (2C, T) from S and G; the
    // GN2 affine per channel, LayerScale folded into the value half.
    {
        double sz = 0.0, sz2 = 0.0;
        const int o = tid;
        double ws = 0.0;
        if (o < 2 * C) {
            double w[H];
#pragma unroll
            for (int h = 0; h < H; ++h) w[h] = (double)L.w2[o * H + h];
            double quad = 0.0;
            int k = H;
#pragma unroll
            for (int h = 0; h < H; ++h) {
                ws += w[h] * sg[h];
                quad += w[h] * w[h] * sg[k++];
#pragma unroll
                for (int h2 = h + 1; h2 < H; ++h2) quad += 2.0 * w[h] * w[h2] * sg[k++];
            }
            const double b = L.b2[o];
            sz = ws + (double)T * b;
            sz2 = quad + 2.0 * b * ws + (double)T * b * b;
        }
        block_sum2(sz, sz2, wsum + 2 * (RW_THREADS / 64));
        if (o < 2 * C) {
            const double cnt = 2.0 * C * (double)T;
            const double m = sz / cnt;
            const float mean = (float)m, inv = 1.0f / (float)sqrt(fmax(sz2 / cnt - m * m, 0.0) + 1e-5);
            const float sc = inv * L.n2w[o], sh = L.n2b[o] + (L.b2[o] - mean) * sc;
            float2 *cf = reinterpret_cast<float2 *>(coef) + (o < C ? 2 * o : 2 * (o - C) + 1);
            if (o < C) {
                const float gm = L.gamma[o];
                *cf = make_float2(sc * gm, sh * gm);
            } else {
                *cf = make_float2(sc, sh);
            }
        }
        __syncthreads();
    }
    // z = W2 g, GN2, GLU, LayerScale, += into the row, channels [grp CG, grp CG + CG).
    if (live) {
        float g[H];
#pragma unroll
        for (int h = 0; h < H; ++h) g[h] = gs[h * TG + t];
        float *xc = xs + grp * CG * S + t + RW_PAD;
        const float *w2 = Lay::WL ? w2s : L.w2;
#pragma unroll 2
        for (int c = grp * CG; c < grp * CG + CG; ++c, xc += S) {
            const float *wv = w2 + c * H, *wg = w2 + (C + c) * H;
            float v = 0.0f, u = 0.0f;
#pragma unroll
            for (int h = 0; h < H; ++h) {
                v = fmaf(wv[h], g[h], v);
                u = fmaf(wg[h], g[h], u);
            }
            const float4 k = coef[c];
            *xc = fmaf(fmaf(v, k.x, k.y), fast_sigmoid(fmaf(u, k.z, k.w)), *xc);
        }
    }
    __syncthreads();
}

// Two workgroups per CU when two rows fit in LDS (C = 48): 6 waves per SIMD.
template <int C, int H>
__global__ __launch_bounds__(RW_THREADS) __attribute__((amdgpu_waves_per_eu(C <= 48 ? 6 : 3)))
void dconv_rows_kernel(float *__restrict__ x, int F, int T, const RowLayers P) {
    static_assert(H % RW_GROUPS == 0 && C % RW_GROUPS == 0, "groups split H and C evenly");
    static_assert(2 * C <= RW_THREADS && RowLds<C, H>::NS <= RW_THREADS, "one thread per GN2 channel / term");
    extern __shared__ __align__(16) char lds[];
    using Lay = RowLds<C, H>;
    float *xs = reinterpret_cast<float *>(lds + Lay::xs);
    const int S = T + 2 * RW_PAD;
    const int z = blockIdx.x, b = z / F, f = z - b * F;
    float *xr = x + ((int64_t)b * C * F + f) * T;
    const int64_t cs = (int64_t)F * T;
    // Row in, halo zeroed.
    if ((T & 3) == 0)
        row_copy<C, 4, true>(xr, cs, xs, S, T);
    else
        row_copy<C, 1, true>(xr, cs, xs, S, T);
    for (int i = threadIdx.x; i < C * 2 * RW_PAD; i += RW_THREADS) {
        const int c = i / (2 * RW_PAD), e = i - c * 2 * RW_PAD;
        xs[c * S + (e < RW_PAD ? e : T + e)] = 0.0f;
    }
    __syncthreads();
    row_layer<C, H>(lds, T, 1, P.l[0]);
    row_layer<C, H>(lds, T, 2, P.l[1]);
    if ((T & 3) == 0)
        row_copy<C, 4, false>(xr, cs, xs, S, T);
    else
        row_copy<C, 1, false>(xr, cs, xs, S, T);
}

template <int C, int H>
bool launch_rows(hipStream_t s, float *x, int B, int F, int T, const RowLayers &P) {
    const int bytes = RowLds<C, H>::bytes(T);
    if (T < 1 || T > RW_TMAX || bytes > RW_LDS_BYTES) return false;
    if (RowLds<C, H>::WL && ((reinterpret_cast<uintptr_t>(P.l[0].w2) | reinterpret_cast<uintptr_t>(P.l[1].w2)) & 15))
        return false;  // W2 is copied to LDS as float4
    static const bool lds_ok = hipFuncSetAttribute(reinterpret_cast<const void *>(&dconv_rows_kernel<C, H>),
                                                   hipFuncAttributeMaxDynamicSharedMemorySize,
                                                   RW_LDS_BYTES) == hipSuccess;
    if (!lds_ok) {
        (void)hipGetLastError();
        return false;
    }
    hipLaunchKernelGGL((dconv_rows_kernel<C, H>), dim3((unsigned)(B * F)), dim3(RW_THREADS), bytes, s, x, F, T, P);
    DMX_LAUNCH_CHECK();
    return true;
}

}  // namespace

int64_t dconv_hidden_floats(int rows, int H, int T) {
    // y, conv1 partials, GN1 affine, Gram partials, GN2 affine, transposed W1
    // (the narrow path's layout; the wide path uses y alone).
    const int C = 8 * H;
    const int64_t items64 = (int64_t)rows * ceil_div(T, C1_POS);
    const int64_t items_g = (int64_t)rows * ceil_div(T, C1_POS * GR_ITER);
    return (int64_t)rows * H * T + 2 * items64 + (int64_t)rows * H * 2 + items_g * (H + H * (H + 1) / 2) +
           (int64_t)rows * 2 * C * 2 + (int64_t)C * 3 * H;
}

void dconv_w1_transposed(const float *w1, int C, int H, float *w1_t) {
    for (int h = 0; h < H; ++h)
        for (int ck = 0; ck < C * 3; ++ck) w1_t[(int64_t)ck * H + h] = w1[(int64_t)h * C * 3 + ck];
}

bool dconv_rows(hipStream_t s, float *x, int B, int C, int F, int T, int H, const DConvRowLayer layers[2]) {
    const RowLayers P{{layers[0], layers[1]}};
    if (H == 6 && C == 48) return launch_rows<48, 6>(s, x, B, F, T, P);
    if (H == 12 && C == 96) return launch_rows<96, 12>(s, x, B, F, T, P);
    return false;
}

bool dconv_narrow_applies(int C, int H) { return (H == 6 && C == 48) || (H == 12 && C == 96); }

bool dconv_layer_narrow(hipStream_t s, float *x, int B, int C, int F, int T, int dil, const float *w1,
                        const float *w1_t, const float *b1, int H, const float *n1w, const float *n1b,
                        const float *w2, const float *b2, const float *n2w, const float *n2b, const float *gamma,
                        float *hbuf) {
    if (H == 6 && C == 48)
        launch_all<48, 6>(s, x, B, F, T, dil, w1, w1_t, b1, n1w, n1b, w2, b2, n2w, n2b, gamma, hbuf);
    else if (H == 12 && C == 96)
        launch_all<96, 12>(s, x, B, F, T, dil, w1, w1_t, b1, n1w, n1b, w2, b2, n2w, n2b, gamma, hbuf);
    else
        return false;
    return true;
}

}  // namespace dmx
