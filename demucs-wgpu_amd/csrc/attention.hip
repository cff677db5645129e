// attention.hip — fused multi-head attention for the cross-transformer:
// softmax(q k^T * scale) v per (batch, head), d_head = 64, fp32 MFMA.
//
// Semantics: `attention_head` (crates/demucs-core/src/demucs/ops.rs:1350-1408):
// scaled = q * scale; S = scaled k^T; P = exp(S - rowmax); O = P v / rowsum.
// Here the row max is the running max over key tiles (online softmax), so the
// Lq x Lk score matrix (231 MB per (b, h) for 2688^2 on the reference device)
// never exists; results agree to f32 rounding.
//
// CDNA4 layout. A workgroup = 4 waves = 128 queries of one (batch, head); each
// wave owns 32 queries. Keys stream through LDS in tiles of 64 (K and V,
// prefetched into registers during the previous tile's math).
//   * Scores are computed transposed, S^T = K Q^T, with v_mfma_f32_32x32x2f32:
//     lane l then holds query l%32 for 32 keys in registers, so row max / row
//     sum need only in-lane reductions plus one cross-half shuffle.
//   * Those score registers are directly the B operand of O^T = V^T P^T: the
//     key contraction order is chosen to match the D-register layout, so P
//     never leaves registers.
//   * The d contraction of QK^T pairs dim s with lane half 0 and dim 32+s with
//     lane half 1, so each lane's Q fragment is one contiguous 32-float run.
#include "common.h"
#include "ops.h"

namespace dmx {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int ATT_D = 64;
constexpr int ATT_KT = 64;      // keys per tile
constexpr int ATT_QW = 32;      // queries per wave
constexpr int ATT_WAVES = 4;
constexpr int ATT_LD = ATT_D + 1;

__global__ __launch_bounds__(256) void attention_kernel(const float *__restrict__ q, int64_t ldq,
                                                        const float *__restrict__ k, int64_t ldk,
                                                        const float *__restrict__ v, int64_t ldv,
                                                        float *__restrict__ out, int64_t ldo, int n_q, int n_k,
                                                        float scale, int64_t q_bs, int64_t kv_bs, int64_t o_bs) {
    __shared__ float Ks[ATT_KT][ATT_LD];
    __shared__ float Vs[ATT_KT][ATT_LD];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int head = blockIdx.y, b = blockIdx.z;
    const int j = lane & 31, half = lane >> 5;
    const int qi = blockIdx.x * (ATT_QW * ATT_WAVES) + wave * ATT_QW + j;
    const bool q_ok = qi < n_q;

    const float *qb = q + b * q_bs + head * ATT_D;
    const float *kb = k + b * kv_bs + head * ATT_D;
    const float *vb = v + b * kv_bs + head * ATT_D;

    // Q fragment: dims [32*half, 32*half + 32) of this lane's query, pre-scaled.
    float qreg[32];
    {
        const float *row = qb + (int64_t)(q_ok ? qi : 0) * ldq + 32 * half;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float4 t = q_ok ? *reinterpret_cast<const float4 *>(row + 4 * i) : make_float4(0.f, 0.f, 0.f, 0.f);
            qreg[4 * i + 0] = t.x * scale;
            qreg[4 * i + 1] = t.y * scale;
            qreg[4 * i + 2] = t.z * scale;
            qreg[4 * i + 3] = t.w * scale;
        }
    }

    // K/V tile staging: 64 keys x 64 dims each = 1024 float4 per tensor, 4 per thread.
    float4 kpre[4], vpre[4];
    auto fetch = [&](int key0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            int e = tid + 256 * i, key = e >> 4, d4 = e & 15;
            int kk = key0 + key;
            if (kk < n_k) {
                kpre[i] = *reinterpret_cast<const float4 *>(kb + (int64_t)kk * ldk + 4 * d4);
                vpre[i] = *reinterpret_cast<const float4 *>(vb + (int64_t)kk * ldv + 4 * d4);
            } else {
                kpre[i] = make_float4(0.f, 0.f, 0.f, 0.f);
                vpre[i] = make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
    };
    auto stage = [&]() {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            int e = tid + 256 * i, key = e >> 4, d = 4 * (e & 15);
            Ks[key][d + 0] = kpre[i].x;
            Ks[key][d + 1] = kpre[i].y;
            Ks[key][d + 2] = kpre[i].z;
            Ks[key][d + 3] = kpre[i].w;
            Vs[key][d + 0] = vpre[i].x;
            Vs[key][d + 1] = vpre[i].y;
            Vs[key][d + 2] = vpre[i].z;
            Vs[key][d + 3] = vpre[i].w;
        }
    };

    floatx16 o0, o1;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        o0[r] = 0.0f;
        o1[r] = 0.0f;
    }
    float m_run = -INFINITY, l_run = 0.0f;

    const int tiles = (n_k + ATT_KT - 1) / ATT_KT;
    fetch(0);
    stage();
    __syncthreads();
    for (int t = 0; t < tiles; ++t) {
        const int key0 = t * ATT_KT;
        if (t + 1 < tiles) fetch(key0 + ATT_KT);

        // S^T for keys [key0, key0+32) and [key0+32, key0+64).
        floatx16 s0, s1;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            s0[r] = 0.0f;
            s1[r] = 0.0f;
        }
#pragma unroll
        for (int s = 0; s < 32; ++s) {
            float a0 = Ks[j][32 * half + s];
            float a1 = Ks[32 + j][32 * half + s];
            s0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, qreg[s], s0, 0, 0, 0);
            s1 = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, qreg[s], s1, 0, 0, 0);
        }
        // Register r of lane l holds key key0 + tile*32 + 8*(r/4) + 4*half + r%4.
        float mloc = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            int kk = key0 + 8 * (r >> 2) + 4 * half + (r & 3);
            if (kk >= n_k) s0[r] = -INFINITY;
            if (kk + 32 >= n_k) s1[r] = -INFINITY;
            mloc = fmaxf(mloc, fmaxf(s0[r], s1[r]));
        }
        mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
        const float m_new = fmaxf(m_run, mloc);
        const float corr = expf(m_run - m_new);
        float lsum = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            s0[r] = expf(s0[r] - m_new);
            s1[r] = expf(s1[r] - m_new);
            lsum += s0[r] + s1[r];
        }
        lsum += __shfl_xor(lsum, 32, 64);
        l_run = l_run * corr + lsum;
        m_run = m_new;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            o0[r] *= corr;
            o1[r] *= corr;
        }
        // O^T += V^T P^T, contracting keys in the order the score registers hold them.
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int kr = 8 * (r >> 2) + 4 * half + (r & 3);
            o0 = __builtin_amdgcn_mfma_f32_32x32x2f32(Vs[kr][j], s0[r], o0, 0, 0, 0);
            o1 = __builtin_amdgcn_mfma_f32_32x32x2f32(Vs[kr][32 + j], s0[r], o1, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int kr = 32 + 8 * (r >> 2) + 4 * half + (r & 3);
            o0 = __builtin_amdgcn_mfma_f32_32x32x2f32(Vs[kr][j], s1[r], o0, 0, 0, 0);
            o1 = __builtin_amdgcn_mfma_f32_32x32x2f32(Vs[kr][32 + j], s1[r], o1, 0, 0, 0);
        }
        __syncthreads();
        if (t + 1 < tiles) {
            stage();
            __syncthreads();
        }
    }

    if (!q_ok) return;
    const float inv = l_run > 0.0f ? 1.0f / l_run : 1.0f;
    float *orow = out + b * o_bs + (int64_t)qi * ldo + head * ATT_D;
    // Register r of o0/o1 holds dim (0|32) + 8*(r/4) + 4*half + r%4.
#pragma unroll
    for (int a = 0; a < 4; ++a) {
        float4 w0 = make_float4(o0[4 * a] * inv, o0[4 * a + 1] * inv, o0[4 * a + 2] * inv, o0[4 * a + 3] * inv);
        float4 w1 = make_float4(o1[4 * a] * inv, o1[4 * a + 1] * inv, o1[4 * a + 2] * inv, o1[4 * a + 3] * inv);
        *reinterpret_cast<float4 *>(orow + 8 * a + 4 * half) = w0;
        *reinterpret_cast<float4 *>(orow + 32 + 8 * a + 4 * half) = w1;
    }
}

}  // namespace

void attention(hipStream_t s, const float *q, int64_t ldq, const float *k, int64_t ldk, const float *v, int64_t ldv,
               float *out, int64_t ldo, int batch, int heads, int n_q, int n_k, int d_head, float scale,
               int64_t q_batch_stride, int64_t kv_batch_stride, int64_t out_batch_stride) {
    require_ptrs({q, k, v, out}, "attention");
    DMX_REQUIRE(d_head == ATT_D, "attention: only d_head = 64 is implemented");
    DMX_REQUIRE(n_q > 0 && n_k > 0 && batch > 0 && heads > 0, "attention: empty problem");
    DMX_REQUIRE(ldq % 4 == 0 && ldk % 4 == 0 && ldv % 4 == 0 && ldo % 4 == 0 && q_batch_stride % 4 == 0 &&
                    kv_batch_stride % 4 == 0 && out_batch_stride % 4 == 0,
                "attention: row strides must be multiples of 4 floats");
    DMX_REQUIRE(((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v) |
                  reinterpret_cast<uintptr_t>(out)) &
                 15) == 0,
                "attention: operands must be 16-byte aligned");
    dim3 grid((unsigned)ceil_div(n_q, ATT_QW * ATT_WAVES), (unsigned)heads, (unsigned)batch);
    hipLaunchKernelGGL(attention_kernel, grid, dim3(256), 0, s, q, ldq, k, ldk, v, ldv, out, ldo, n_q, n_k, scale,
                       q_batch_stride, kv_batch_stride, out_batch_stride);
    DMX_LAUNCH_CHECK();
}

}  // namespace dmx
