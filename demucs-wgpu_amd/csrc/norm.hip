// norm.hip — LayerNorm, GroupNorm and the elementwise ops of the forward.
// HBM-bound: each kernel reads and writes its tensor once, float4 where the
// layout allows, with wave64 shuffle reductions.

#include "common.h"
#include "ops.h"

namespace dmx {
namespace {

// `layer_norm_rows` (crates/demucs-core/src/demucs/ops.rs:596-621): f32 mean,
// f32 biased variance about it, inv = 1/sqrt(var + 1e-5);
// out = (x - mean) * inv * w + b (+ add[row % add_rows]). One wave per row.
__global__ __launch_bounds__(256) void layer_norm_kernel(const float *__restrict__ x, int rows, int dim,
                                                         const float *__restrict__ w, const float *__restrict__ b,
                                                         float *__restrict__ out, const float *__restrict__ add,
                                                         int add_rows) {
    int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float *xr = x + (int64_t)row * dim;
    float s = 0.0f;
    for (int i = lane; i < dim; i += 64) s += xr[i];
    float mean = wave_sum(s) / (float)dim;
    float v = 0.0f;
    for (int i = lane; i < dim; i += 64) {
        float d = xr[i] - mean;
        v += d * d;
    }
    float var = wave_sum(v) / (float)dim;
    float inv = 1.0f / sqrtf(var + 1e-5f);
    float *orow = out + (int64_t)row * dim;
    const float *ar = add ? add + (int64_t)(row % add_rows) * dim : nullptr;
    for (int i = lane; i < dim; i += 64) {
        float y = (xr[i] - mean) * inv * w[i] + b[i];
        if (ar) y += ar[i];
        orow[i] = y;
    }
}

// The same for dim = 4 * 64 * V (the model's 512: V = 2), row held in
// registers: one read and one write of the row, float4 wide. Same two-pass
// arithmetic (mean, then the mean of squared deviations).
template <int V>
__global__ __launch_bounds__(256) void layer_norm_vec_kernel(const float4 *__restrict__ x, int rows,
                                                             const float4 *__restrict__ w,
                                                             const float4 *__restrict__ b, float4 *__restrict__ out,
                                                             const float4 *__restrict__ add, int add_rows) {
    constexpr int DIM4 = 64 * V;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float4 *xr = x + (int64_t)row * DIM4;
    float4 v[V];
#pragma unroll
    for (int j = 0; j < V; ++j) v[j] = xr[lane + 64 * j];
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < V; ++j) s += (v[j].x + v[j].y) + (v[j].z + v[j].w);
    const float mean = wave_sum(s) / (float)(4 * DIM4);
    float q = 0.0f;
#pragma unroll
    for (int j = 0; j < V; ++j) {
        const float a = v[j].x - mean, c = v[j].y - mean, d = v[j].z - mean, e = v[j].w - mean;
        q += (a * a + c * c) + (d * d + e * e);
    }
    const float var = wave_sum(q) / (float)(4 * DIM4);
    const float inv = 1.0f / sqrtf(var + 1e-5f);
    float4 *orow = out + (int64_t)row * DIM4;
    const float4 *ar = add ? add + (int64_t)(row % add_rows) * DIM4 : nullptr;
#pragma unroll
    for (int j = 0; j < V; ++j) {
        const int i = lane + 64 * j;
        const float4 wv = w[i], bv = b[i];
        float4 y = make_float4((v[j].x - mean) * inv * wv.x + bv.x, (v[j].y - mean) * inv * wv.y + bv.y,
                               (v[j].z - mean) * inv * wv.z + bv.z, (v[j].w - mean) * inv * wv.w + bv.w);
        if (ar) {
            const float4 av = ar[i];
            y = make_float4(y.x + av.x, y.y + av.y, y.z + av.z, y.w + av.w);
        }
        orow[i] = y;
    }
}

// layer_norm_vec_kernel with the normalised row written as P bf16 planes
// (plane q of element i of row r at out + q * stride + r * 4 * DIM4 + i), for
// the transformer linears that read it.
template <int V, int P>
__global__ __launch_bounds__(256) void layer_norm_planes_kernel(const float4 *__restrict__ x, int rows,
                                                                const float4 *__restrict__ w,
                                                                const float4 *__restrict__ b,
                                                                unsigned short *__restrict__ out, int64_t stride) {
    constexpr int DIM4 = 64 * V;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float4 *xr = x + (int64_t)row * DIM4;
    float4 v[V];
#pragma unroll
    for (int j = 0; j < V; ++j) v[j] = xr[lane + 64 * j];
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < V; ++j) s += (v[j].x + v[j].y) + (v[j].z + v[j].w);
    const float mean = wave_sum(s) / (float)(4 * DIM4);
    float q = 0.0f;
#pragma unroll
    for (int j = 0; j < V; ++j) {
        const float a = v[j].x - mean, c = v[j].y - mean, d = v[j].z - mean, e = v[j].w - mean;
        q += (a * a + c * c) + (d * d + e * e);
    }
    const float var = wave_sum(q) / (float)(4 * DIM4);
    const float inv = 1.0f / sqrtf(var + 1e-5f);
    unsigned short *orow = out + (int64_t)row * 4 * DIM4;
#pragma unroll
    for (int j = 0; j < V; ++j) {
        const int i = lane + 64 * j;
        const float4 wv = w[i], bv = b[i];
        const float4 y = make_float4((v[j].x - mean) * inv * wv.x + bv.x, (v[j].y - mean) * inv * wv.y + bv.y,
                                     (v[j].z - mean) * inv * wv.z + bv.z, (v[j].w - mean) * inv * wv.w + bv.w);
        store_planes4<P>(orow + 4 * i, stride, y);
    }
}

// x -> P bf16 planes, four values per thread.
template <int P>
__global__ __launch_bounds__(256) void split_planes_kernel(const float *__restrict__ x, int64_t n,
                                                           unsigned short *__restrict__ out, int64_t stride) {
    const int64_t i = 4 * ((int64_t)blockIdx.x * 256 + threadIdx.x);
    if (i + 3 < n) {
        store_planes4<P>(out + i, stride, *reinterpret_cast<const float4 *>(x + i));
    } else {
        for (int64_t e = i; e < n; ++e) store_planes1<P>(out + e, stride, x[e]);
    }
}

// (b, c, F*T) channel-major -> LayerNorm'd token rows (b, T*F, c), token = t*F + f,
// plus pos[token] * pos_weight. A block stages TOK_POS positions x all
// channels in LDS ([c][TOK_POS + 1]: an odd row stride, so a wave reading one
// position across 64 channels hits 64 distinct banks), reading each channel's
// run of TOK_POS floats as float4s, then writes whole token rows. Blocks are handed to the 8 XCDs round-robin; the work list is
// (position block, batch row) with the batch row fastest and each XCD takes a
// contiguous range of it, so the batch rows of a position block run on one
// XCD and read that block's positional rows into one L2.
constexpr int TOK_XCDS = 8;
// CK = c / 64 when c is a multiple of 64 up to 512 (the model's 512: CK = 8):
// each lane keeps its CK channels' weights, biases and values in registers
// and issues a position's CK positional loads together; CK = 0 is the
// general loop for any c.
template <int TOK_POS, int NT, int CK>
__global__ __launch_bounds__(NT) void channels_to_tokens_ln_kernel(const float *__restrict__ x, int B, int c, int F,
                                                                   int T, const float *__restrict__ w,
                                                                   const float *__restrict__ bias,
                                                                   const float *__restrict__ pos, float pos_weight,
                                                                   float *__restrict__ out) {
    extern __shared__ float tile[];  // [c][TOK_POS + 1]
    constexpr int S = TOK_POS + 1, Q = TOK_POS / 4, WAVES = NT / 64;
    const int P = F * T, NP = (P + TOK_POS - 1) / TOK_POS;
    const int items = NP * B, per_xcd = (items + TOK_XCDS - 1) / TOK_XCDS;
    const int item = (int)(blockIdx.x % TOK_XCDS) * per_xcd + (int)(blockIdx.x / TOK_XCDS);
    if (item >= items || (int)(blockIdx.x / TOK_XCDS) >= per_xcd) return;
    const int b = item % B, p0 = (item / B) * TOK_POS;
    const float *xb = x + (int64_t)b * c * P;
    if ((P & 3) == 0 && p0 + TOK_POS <= P) {
        for (int e = threadIdx.x; e < c * Q; e += NT) {
            const int ch = e / Q, q = e - ch * Q;
            const float4 v = *reinterpret_cast<const float4 *>(xb + (int64_t)ch * P + p0 + 4 * q);
            float *t = tile + ch * S + 4 * q;
            t[0] = v.x;
            t[1] = v.y;
            t[2] = v.z;
            t[3] = v.w;
        }
    } else {
        for (int e = threadIdx.x; e < c * TOK_POS; e += NT) {
            const int ch = e / TOK_POS, pi = e - ch * TOK_POS, p = p0 + pi;
            tile[ch * S + pi] = p < P ? xb[(int64_t)ch * P + p] : 0.0f;
        }
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if constexpr (CK > 0) {
        float wv[CK], bv[CK];
#pragma unroll
        for (int k = 0; k < CK; ++k) {
            wv[k] = w[lane + 64 * k];
            bv[k] = bias[lane + 64 * k];
        }
        __syncthreads();
        for (int pi = wave; pi < TOK_POS; pi += WAVES) {
            const int p = p0 + pi;
            if (p >= P) break;
            const int f = p / T, t = p - f * T, token = t * F + f;
            float pv[CK];
            const float *prow = pos ? pos + (int64_t)token * c : nullptr;
#pragma unroll
            for (int k = 0; k < CK; ++k) pv[k] = prow ? prow[lane + 64 * k] : 0.0f;
            float xv[CK];
            float s = 0.0f;
#pragma unroll
            for (int k = 0; k < CK; ++k) {
                xv[k] = tile[(lane + 64 * k) * S + pi];
                s += xv[k];
            }
            const float mean = wave_sum(s) / (float)c;
            float v = 0.0f;
#pragma unroll
            for (int k = 0; k < CK; ++k) {
                const float d = xv[k] - mean;
                v += d * d;
            }
            const float var = wave_sum(v) / (float)c;
            const float inv = 1.0f / sqrtf(var + 1e-5f);
            float *orow = out + ((int64_t)b * P + token) * c;
#pragma unroll
            for (int k = 0; k < CK; ++k) {
                float y = (xv[k] - mean) * inv * wv[k] + bv[k];
                if (prow) y = y + pv[k] * pos_weight;
                orow[lane + 64 * k] = y;
            }
        }
    } else {
        __syncthreads();
        for (int pi = wave; pi < TOK_POS; pi += WAVES) {
            const int p = p0 + pi;
            if (p >= P) break;
            float s = 0.0f;
            for (int ch = lane; ch < c; ch += 64) s += tile[ch * S + pi];
            const float mean = wave_sum(s) / (float)c;
            float v = 0.0f;
            for (int ch = lane; ch < c; ch += 64) {
                const float d = tile[ch * S + pi] - mean;
                v += d * d;
            }
            const float var = wave_sum(v) / (float)c;
            const float inv = 1.0f / sqrtf(var + 1e-5f);
            const int f = p / T, t = p - f * T, token = t * F + f;
            float *orow = out + ((int64_t)b * P + token) * c;
            const float *prow = pos ? pos + (int64_t)token * c : nullptr;
            for (int ch = lane; ch < c; ch += 64) {
                float y = (tile[ch * S + pi] - mean) * inv * w[ch] + bias[ch];
                if (prow) y = y + prow[ch] * pos_weight;
                orow[ch] = y;
            }
        }
    }
}

// MyGroupNorm(1, C) on token planes (crates/demucs-core/src/demucs/host.rs:1137-1196):
// scale = inv * w[c], shift = bias[c] - mean * scale, x = x * scale + shift.
// The grid stride is a multiple of the row's C/4 float4s, so each thread keeps
// one channel quad: its scale and shift are computed once, and the loop is a
// float4 load, four FMAs and a store, GN_UNROLL loads in flight.
constexpr int GN_UNROLL = 4;
__global__ __launch_bounds__(256) void gn_tokens_apply_kernel(float4 *__restrict__ x, int64_t per_batch4, int C4,
                                                              const double *__restrict__ stats, double count,
                                                              const float4 *__restrict__ w,
                                                              const float4 *__restrict__ bias) {
    const int b = blockIdx.y;
    float mean, inv;
    gn_stats(stats + 2 * b, count, mean, inv);
    float4 *xb = x + b * per_batch4;
    const int64_t start = (int64_t)blockIdx.x * 256 + threadIdx.x, stride = (int64_t)gridDim.x * 256;
    const int c4 = (int)(start % C4);
    const float4 ww = w[c4], bb = bias[c4];
    const float4 sc = make_float4(inv * ww.x, inv * ww.y, inv * ww.z, inv * ww.w);
    const float4 sh = make_float4(bb.x - mean * sc.x, bb.y - mean * sc.y, bb.z - mean * sc.z, bb.w - mean * sc.w);
    auto apply = [&](float4 v) {
        return make_float4(fmaf(v.x, sc.x, sh.x), fmaf(v.y, sc.y, sh.y), fmaf(v.z, sc.z, sh.z), fmaf(v.w, sc.w, sh.w));
    };
    if (stride % C4 != 0) {  // the channel quad changes along the loop
        for (int64_t i = start; i < per_batch4; i += stride) {
            const int q = (int)(i % C4);
            const float4 wq = w[q], bq = bias[q], v = xb[i];
            xb[i] = make_float4(fmaf(v.x, inv * wq.x, bq.x - mean * inv * wq.x),
                                fmaf(v.y, inv * wq.y, bq.y - mean * inv * wq.y),
                                fmaf(v.z, inv * wq.z, bq.z - mean * inv * wq.z),
                                fmaf(v.w, inv * wq.w, bq.w - mean * inv * wq.w));
        }
        return;
    }
    int64_t i = start;
    for (; i + (GN_UNROLL - 1) * stride < per_batch4; i += GN_UNROLL * stride) {
        float4 v[GN_UNROLL];
#pragma unroll
        for (int u = 0; u < GN_UNROLL; ++u) v[u] = xb[i + u * stride];
#pragma unroll
        for (int u = 0; u < GN_UNROLL; ++u) xb[i + u * stride] = apply(v[u]);
    }
    for (; i < per_batch4; i += stride) xb[i] = apply(xb[i]);
}

// f64 moments of each (batch, group) run of `len` floats.
__global__ __launch_bounds__(256) void moments_kernel(const float *__restrict__ x, int64_t len,
                                                      double *__restrict__ stats) {
    const float *p = x + (int64_t)blockIdx.y * len;
    double s = 0.0, q = 0.0;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < len; i += (int64_t)gridDim.x * 256) {
        double v = p[i];
        s += v;
        q += v * v;
    }
    block_moments_atomic(s, q, stats + 2 * blockIdx.y);
}

// `group_norm` apply (demucs/ops.rs:583-589).
__global__ __launch_bounds__(256) void group_norm_apply_kernel(const float *__restrict__ x, int c, int64_t inner,
                                                               int groups, const float *__restrict__ w,
                                                               const float *__restrict__ bias,
                                                               const double *__restrict__ stats,
                                                               float *__restrict__ out, int64_t total) {
    int per_group = c / groups;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        int64_t bc = i / inner;
        int ch = (int)(bc % c);
        int64_t b = bc / c;
        int g = ch / per_group;
        float mean, inv;
        gn_stats(stats + 2 * (b * groups + g), (double)per_group * (double)inner, mean, inv);
        float scale = inv * w[ch];
        float shift = bias[ch] - mean * scale;
        out[i] = x[i] * scale + shift;
    }
}

// `glu` (demucs/ops.rs:624-658).
__global__ __launch_bounds__(256) void glu_kernel(const float *__restrict__ x, int c, int64_t inner,
                                                  float *__restrict__ out, int64_t total) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        int64_t row = i / inner, t = i - row * inner;
        int64_t b = row / c, ch = row % c;
        const float *value = x + (b * 2 * c + ch) * inner;
        out[i] = value[t] * sigmoid(value[c * inner + t]);
    }
}

__global__ __launch_bounds__(256) void gelu_kernel(const float *__restrict__ x, int64_t n, float *__restrict__ out) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) out[i] = gelu(x[i]);
}

__global__ __launch_bounds__(256) void zero_f_kernel(float *p, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) p[i] = 0.0f;
}

__global__ __launch_bounds__(256) void copy_rows_kernel(const float *__restrict__ src, int64_t src_ld, int64_t n_copy,
                                                        float *__restrict__ dst, int64_t dst_len) {
    const int64_t r = blockIdx.y;
    for (int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x; t < dst_len; t += (int64_t)gridDim.x * 256)
        dst[r * dst_len + t] = t < n_copy ? src[r * src_ld + t] : 0.0f;
}

__global__ __launch_bounds__(256) void zero_kernel(double *p, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) p[i] = 0.0;
}

unsigned grid_for(int64_t n, int64_t cap = 8192) {
    int64_t g = ceil_div(n, 256);
    return (unsigned)std::max<int64_t>(1, std::min<int64_t>(g, cap));
}

}  // namespace

void layer_norm_rows(hipStream_t s, const float *x, int rows, int dim, const float *w, const float *b, float *out,
                     const float *add, int add_rows) {
    if (rows <= 0) return;
    require_ptrs({x, w, b, out}, "layer_norm_rows");
    DMX_REQUIRE(!add || add_rows > 0, "layer_norm_rows: add needs a row count");
    const bool vec = ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(b) |
                       reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(add)) &
                      15) == 0;
    if (vec && dim == 512) {
        hipLaunchKernelGGL(layer_norm_vec_kernel<2>, dim3((unsigned)ceil_div(rows, 4)), dim3(256), 0, s,
                           reinterpret_cast<const float4 *>(x), rows, reinterpret_cast<const float4 *>(w),
                           reinterpret_cast<const float4 *>(b), reinterpret_cast<float4 *>(out),
                           reinterpret_cast<const float4 *>(add), add ? add_rows : 1);
    } else {
        hipLaunchKernelGGL(layer_norm_kernel, dim3((unsigned)ceil_div(rows, 4)), dim3(256), 0, s, x, rows, dim, w, b,
                           out, add, add ? add_rows : 1);
    }
    DMX_LAUNCH_CHECK();
}

void layer_norm_planes(hipStream_t s, const float *x, int rows, int dim, const float *w, const float *b, Planes out) {
    if (rows <= 0) return;
    require_ptrs({x, w, b, out.p}, "layer_norm_planes");
    DMX_REQUIRE(dim == 512, "layer_norm_planes: rows of 512 only");
    DMX_REQUIRE(((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(b)) &
                 15) == 0 && (reinterpret_cast<uintptr_t>(out.p) & 7) == 0 && out.stride % 4 == 0,
                "layer_norm_planes: operands must be aligned");
    DMX_REQUIRE(out.count == 1 || out.count == 3, "layer_norm_planes: 1 or 3 planes");
    DMX_REQUIRE(out.count == 1 || out.stride >= (int64_t)rows * dim, "layer_norm_planes: planes overlap");
    auto go = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, dim3((unsigned)ceil_div(rows, 4)), dim3(256), 0, s,
                           reinterpret_cast<const float4 *>(x), rows, reinterpret_cast<const float4 *>(w),
                           reinterpret_cast<const float4 *>(b), out.p, out.stride);
    };
    if (out.count == 3)
        go(layer_norm_planes_kernel<2, 3>);
    else
        go(layer_norm_planes_kernel<2, 1>);
    DMX_LAUNCH_CHECK();
}

void split_to_planes(hipStream_t s, const float *x, int64_t n, Planes out) {
    if (n <= 0) return;
    require_ptrs({x, out.p}, "split_to_planes");
    DMX_REQUIRE(((reinterpret_cast<uintptr_t>(x) & 15) | (reinterpret_cast<uintptr_t>(out.p) & 7)) == 0 &&
                    out.stride % 4 == 0,
                "split_to_planes: operands must be aligned");
    DMX_REQUIRE(out.count == 1 || out.count == 3, "split_to_planes: 1 or 3 planes");
    DMX_REQUIRE(out.count == 1 || out.stride >= n, "split_to_planes: planes overlap");
    const unsigned blocks = (unsigned)ceil_div(ceil_div(n, (int64_t)4), (int64_t)256);
    if (out.count == 3)
        hipLaunchKernelGGL(split_planes_kernel<3>, dim3(blocks), dim3(256), 0, s, x, n, out.p, out.stride);
    else
        hipLaunchKernelGGL(split_planes_kernel<1>, dim3(blocks), dim3(256), 0, s, x, n, out.p, out.stride);
    DMX_LAUNCH_CHECK();
}

template <int TOK_POS, int NT>
void launch_tokens_ln(hipStream_t s, const float *x, int b, int c, int F, int T, const float *w, const float *bias,
                      const float *pos, float pos_weight, float *out) {
    const size_t shmem = (size_t)c * (TOK_POS + 1) * sizeof(float);
    constexpr size_t LDS_MAX = 96 * 1024;
    DMX_REQUIRE(shmem <= LDS_MAX, "channels_to_tokens_ln: too many channels");
    const int64_t items = ceil_div((int64_t)F * T, TOK_POS) * b;
    const int64_t per_xcd = ceil_div(items, TOK_XCDS);
    auto go = [&](auto kernel) {
        static const bool lds_ok = hipFuncSetAttribute(reinterpret_cast<const void *>(kernel),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                                       (int)LDS_MAX) == hipSuccess;
        DMX_REQUIRE(lds_ok, "channels_to_tokens_ln: the kernel's LDS limit could not be raised");
        hipLaunchKernelGGL(kernel, dim3((unsigned)(per_xcd * TOK_XCDS)), dim3(NT), shmem, s, x, b, c, F, T, w, bias,
                           pos, pos_weight, out);
    };
    if (c == 512)
        go(channels_to_tokens_ln_kernel<TOK_POS, NT, 8>);
    else
        go(channels_to_tokens_ln_kernel<TOK_POS, NT, 0>);
    DMX_LAUNCH_CHECK();
}

void channels_to_tokens_ln(hipStream_t s, const float *x, int b, int c, int F, int T, const float *w,
                           const float *bias, const float *pos, float pos_weight, float *out) {
    require_ptrs({x, w, bias, out}, "channels_to_tokens_ln");
    // Eight positions per block: a channel row's run is 32 B (two float4),
    // the LDS tile 17 KB, and every wave writes two token rows. Measured at
    // B = 8, c = 512 (2688 and 1344 tokens): 23 and 13 us; blocks of 16 and
    // 32 positions took 26 and 34 us, since a block's rows are written one
    // position per wave after its loads.
    launch_tokens_ln<8, 256>(s, x, b, c, F, T, w, bias, pos, pos_weight, out);
}

void group_norm_tokens_apply(hipStream_t s, float *x, int b, int L, int C, const double *stats, const float *w,
                             const float *bias) {
    require_ptrs({x, stats, w, bias}, "group_norm_tokens_apply");
    DMX_REQUIRE(C % 4 == 0, "group_norm_tokens_apply: channels must be a multiple of 4");
    int64_t per4 = (int64_t)L * C / 4;
    // About 8 float4 per thread; a stride that keeps each thread on one channel
    // quad when C/4 divides 256 (C = 512: 128 quads).
    const int64_t blocks = std::min<int64_t>(std::max<int64_t>(1, per4 / (256 * 2 * GN_UNROLL)), 65535);
    dim3 grid((unsigned)blocks, (unsigned)b);
    hipLaunchKernelGGL(gn_tokens_apply_kernel, grid, dim3(256), 0, s, reinterpret_cast<float4 *>(x), per4, C / 4,
                       stats, (double)L * (double)C, reinterpret_cast<const float4 *>(w),
                       reinterpret_cast<const float4 *>(bias));
    DMX_LAUNCH_CHECK();
}

void group_norm(hipStream_t s, const float *x, int b, int c, int inner, int groups, const float *w, const float *bias,
                float *out, double *stats) {
    DMX_REQUIRE(groups > 0 && c % groups == 0, "group_norm: channels not divisible by groups");
    int64_t len = (int64_t)(c / groups) * inner;
    zero_doubles(s, stats, 2 * (int64_t)b * groups);
    hipLaunchKernelGGL(moments_kernel, dim3(grid_for(len, 512), (unsigned)(b * groups)), dim3(256), 0, s, x, len,
                       stats);
    DMX_LAUNCH_CHECK();
    int64_t total = (int64_t)b * c * inner;
    hipLaunchKernelGGL(group_norm_apply_kernel, dim3(grid_for(total)), dim3(256), 0, s, x, c, (int64_t)inner, groups,
                       w, bias, stats, out, total);
    DMX_LAUNCH_CHECK();
}

void glu(hipStream_t s, const float *x, int b, int c2, int inner, float *out) {
    DMX_REQUIRE(c2 % 2 == 0, "GLU needs an even channel count");
    int64_t total = (int64_t)b * (c2 / 2) * inner;
    hipLaunchKernelGGL(glu_kernel, dim3(grid_for(total)), dim3(256), 0, s, x, c2 / 2, (int64_t)inner, out, total);
    DMX_LAUNCH_CHECK();
}

void gelu(hipStream_t s, const float *x, int64_t n, float *out) {
    hipLaunchKernelGGL(gelu_kernel, dim3(grid_for(n)), dim3(256), 0, s, x, n, out);
    DMX_LAUNCH_CHECK();
}

void zero_doubles(hipStream_t s, double *p, int64_t n) {
    if (n <= 0) return;
    hipLaunchKernelGGL(zero_kernel, dim3(grid_for(n, 1024)), dim3(256), 0, s, p, n);
    DMX_LAUNCH_CHECK();
}

void zero_floats(hipStream_t s, float *p, int64_t n) {
    if (n <= 0) return;
    hipLaunchKernelGGL(zero_f_kernel, dim3(grid_for(n, 4096)), dim3(256), 0, s, p, n);
    DMX_LAUNCH_CHECK();
}

void copy_rows(hipStream_t s, const float *src, int64_t rows, int64_t src_ld, int64_t n_copy, float *dst,
               int64_t dst_len) {
    if (rows <= 0 || dst_len <= 0) return;
    DMX_REQUIRE(rows <= 65535, "copy_rows: too many rows");
    hipLaunchKernelGGL(copy_rows_kernel, dim3(grid_for(dst_len, 1024), (unsigned)rows), dim3(256), 0, s, src, src_ld,
                       n_copy, dst, dst_len);
    DMX_LAUNCH_CHECK();
}

}  // namespace dmx
