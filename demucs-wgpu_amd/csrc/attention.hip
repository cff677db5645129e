// attention.hip — fused multi-head attention for the cross-transformer:
// softmax(q k^T * scale) v per (batch, head), d_head = 64, fp32 MFMA.
//
// Semantics: `attention_head` (crates/demucs-core/src/demucs/ops.rs:1350-1408):
// scaled = q * scale; S = scaled k^T; P = exp(S - rowmax); O = P v / rowsum.
// Here the row max is a running max over key tiles (online softmax), so the
// Lq x Lk score matrix (231 MB per (b, h) for 2688^2 on the reference device)
// never exists; results agree to f32 rounding.
//
// CDNA4 layout. A workgroup = 4 waves = 128 queries of one (batch, head); each
// wave owns 32 queries. Keys stream through LDS in tiles of 64, double
// buffered: the next tile is fetched into registers while the current one is
// multiplied, then written to the other buffer, so one barrier per tile.
//   * Scores are computed transposed, S^T = K Q^T, with v_mfma_f32_32x32x2f32:
//     lane l then holds query l%32 for 32 keys in registers, so row max / row
//     sum need only in-lane reductions plus one cross-half shuffle.
//   * Those score registers are directly the B operand of O^T = V^T P^T: the
//     key contraction order is chosen to match the D-register layout, so P
//     never leaves registers.
//   * The d contraction of QK^T pairs dim s with lane half 0 and dim 32+s with
//     lane half 1, so each lane's Q fragment is one contiguous 32-float run.
//   * K is kept [key][d] and V transposed [d][key] in LDS, rows padded to 68
//     floats: every MFMA operand then comes from a 128-bit LDS read (4 MFMAs
//     per read), and the reads and the staging writes are bank-conflict free.
//   * Scores live in log2 units (Q is pre-scaled by scale * log2 e), so each
//     probability is one v_exp_f32. The running max is raised lazily: only
//     when some query's tile max exceeds it by more than ATT_SLACK, so the
//     accumulator rescale is skipped on most tiles while exp2(s - m) stays
//     below 2^ATT_SLACK. O and the row sum carry the same factor, which the
//     final division cancels. The score MFMAs accumulate onto -m rather than
//     0, so they deliver s - m and the exponentials need no subtraction.
//   * K/V tiles are fetched through buffer resources (scalar base and size,
//     32-bit lane offsets): no per-tile address arithmetic on the VALU.
//   * The file is compiled with -fno-honor-nans: no NaN reaches the kernels
//     from finite inputs, and the row maxima then take no canonicalising
//     v_max per score.
#include <algorithm>
#include <cstdlib>
#include <type_traits>
#include <utility>

#include "common.h"
#include "ops.h"

// Waves per SIMD the register allocation must leave room for.
#ifndef DMX_ATT_WAVES_PER_EU
#define DMX_ATT_WAVES_PER_EU 2
#endif

namespace dmx {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int ATT_D = 64;
constexpr int ATT_KT = 64;      // keys per tile
constexpr int ATT_QW = 32;      // queries per wave
constexpr int ATT_WAVES = 4;
constexpr int ATT_LD = 68;      // padded LDS row (floats); 16-byte aligned rows
constexpr float ATT_LOG2E = 1.4426950408889634f;
constexpr float ATT_SLACK = 8.0f;

__device__ __forceinline__ float4 lds4(const float *p) { return *reinterpret_cast<const float4 *>(p); }

// A wave raises its issue priority (s_setprio 1) for its two runs of MFMAs
// per tile and drops it for the softmax: when both waves on a SIMD are ready,
// the one feeding the matrix core issues first, and the other's softmax fills
// the matrix core's busy cycles (0.997-1.003 against 1.016 ms per paired
// cross launch). DMX_ATT_SETPRIO=0 builds without it.
#ifndef DMX_ATT_SETPRIO
#define DMX_ATT_SETPRIO 1
#endif
template <int P>
__device__ __forceinline__ void att_prio_imm() {
    __builtin_amdgcn_s_setprio(P);
}
__device__ __forceinline__ void att_prio(int p) {
#if DMX_ATT_SETPRIO
    if (p)
        att_prio_imm<DMX_ATT_SETPRIO>();
    else
        att_prio_imm<0>();
#else
    (void)p;
#endif
}

// Raw buffer resource over `bytes` bytes from `base` (gfx9 word 3: 32-bit
// raw data format). Loads at offsets >= bytes return zeros.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t att_rsrc(const float *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(base), (short)0, (int)bytes, 0x00020000);
}

// One launch covers up to two attention problems (the two branches of a
// transformer layer): blocks [0, p[0].blocks) work on p[0], the rest on p[1].
// A block is 128 queries of one (batch row, head); within a problem the
// query blocks of one (row, head) are adjacent, so their K/V stays in L2.
struct AttProblem {
    const float *q, *k, *v;
    float *out;
    unsigned short *out_planes;  // when set: the output as `planes` bf16 planes, plane_stride apart
    int64_t plane_stride;
    int planes;
    const unsigned short *kp, *vt;  // K / V^T planes (KVPlanes) of the three-plane kernel
    int64_t kp_ps, kp_bs, kp_ld, vt_ps, ldvt;
    int64_t ldq, ldk, ldv, ldo, q_bs, kv_bs, o_bs;
    int n_q, n_k, heads, qblocks, blocks;
};
struct AttGroup {
    AttProblem p[2];
    int count;
    float scale;
};

// Within a problem whose (row, head) pairs split evenly over the 8 XCDs (and
// which starts on XCD 0), XCD x runs all query blocks of pairs x, x + 8, ...:
// a pair's K/V is then read into one L2, and every XCD gets the same share of
// each problem, long-key blocks first.
__device__ __forceinline__ int att_xcd_block(int bid, const AttProblem &P, bool aligned) {
#if DMX_XCD_REMAP
    const int pairs = P.blocks / P.qblocks;
    if (!aligned || pairs % XCDS != 0) return bid;
    const int x = bid % XCDS, local = bid / XCDS;
    return ((local / P.qblocks) * XCDS + x) * P.qblocks + local % P.qblocks;
#else
    (void)P;
    (void)aligned;
    return bid;
#endif
}

// A wave's output rows: lane (query) qi's dims (0|32) + 8 a + 4 half + 0..3
// from o0/o1 registers 4a..4a+3, times inv, at element offset `at` of the
// output (fp32, or bf16 planes).
template <class Acc>
__device__ __forceinline__ void att_store(const AttProblem &P, int64_t at, int half, const Acc &o0, const Acc &o1,
                                          float inv) {
    auto row = [&](int a, int hi) {
        const Acc &o = hi ? o1 : o0;
        return make_float4(o[4 * a] * inv, o[4 * a + 1] * inv, o[4 * a + 2] * inv, o[4 * a + 3] * inv);
    };
    if (P.out_planes) {
        unsigned short *prow = P.out_planes + at;
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
            for (int hi = 0; hi < 2; ++hi) {
                if (P.planes == 3)
                    store_planes4<3>(prow + 32 * hi + 8 * a + 4 * half, P.plane_stride, row(a, hi));
                else
                    store_planes4<1>(prow + 32 * hi + 8 * a + 4 * half, P.plane_stride, row(a, hi));
            }
        return;
    }
    float *orow = P.out + at;
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int hi = 0; hi < 2; ++hi) *reinterpret_cast<float4 *>(orow + 32 * hi + 8 * a + 4 * half) = row(a, hi);
}

// The problem of this block and its (query block, head, batch row).
#define DMX_ATT_LOCATE(g)                                                                          \
    int bid_ = blockIdx.x;                                                                         \
    const int pi_ = ((g).count > 1 && bid_ >= (g).p[0].blocks) ? 1 : 0;                           \
    if (pi_) bid_ -= (g).p[0].blocks;                                                              \
    const AttProblem &P_ = (g).p[pi_];                                                             \
    bid_ = att_xcd_block(bid_, P_, pi_ == 0 || (g).p[0].blocks % XCDS == 0);                       \
    const float *__restrict__ q = P_.q;                                                            \
    const float *__restrict__ k = P_.k;                                                            \
    const float *__restrict__ v = P_.v;                                                            \
    const int64_t ldq = P_.ldq, ldk = P_.ldk, ldv = P_.ldv, ldo = P_.ldo;                          \
    const int64_t q_bs = P_.q_bs, kv_bs = P_.kv_bs, o_bs = P_.o_bs;                                \
    const int n_q = P_.n_q, n_k = P_.n_k;                                                          \
    const float scale = (g).scale;                                                                 \
    const int qblock = bid_ % P_.qblocks, head = (bid_ / P_.qblocks) % P_.heads,                  \
              b = bid_ / (P_.qblocks * P_.heads);

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(DMX_ATT_WAVES_PER_EU)))
void attention_kernel(const AttGroup g) {
    DMX_ATT_LOCATE(g)
    __shared__ __align__(16) float Ks[2][ATT_KT][ATT_LD];  // [buffer][key][d]
    __shared__ __align__(16) float Vt[2][ATT_D][ATT_LD];   // [buffer][d][key]

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int j = lane & 31, half = lane >> 5;
    const int qi = qblock * (ATT_QW * ATT_WAVES) + wave * ATT_QW + j;
    const bool q_ok = qi < n_q;

    const float *qb = q + b * q_bs + head * ATT_D;
    const float *kb = k + b * kv_bs + head * ATT_D;
    const float *vb = v + b * kv_bs + head * ATT_D;

    // Q fragment: dims [32*half, 32*half + 32) of this lane's query, pre-scaled
    // into log2 units.
    float qreg[32];
    {
        const float qs = scale * ATT_LOG2E;
        const float *row = qb + (int64_t)(q_ok ? qi : 0) * ldq + 32 * half;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float4 t = q_ok ? *reinterpret_cast<const float4 *>(row + 4 * i) : make_float4(0.f, 0.f, 0.f, 0.f);
            qreg[4 * i + 0] = t.x * qs;
            qreg[4 * i + 1] = t.y * qs;
            qreg[4 * i + 2] = t.z * qs;
            qreg[4 * i + 3] = t.w * qs;
        }
    }

    // Tile staging: 64 keys x 16 float4 per tensor; slot i of this thread is
    // key 16*(s%4) + lane%16, float4 column 4*(s/4) + lane/16 with s = 4*wave + i.
    // A wave then writes 16 keys x 4 columns at once, which keeps the
    // transposed V writes on 64 distinct banks.
    floatx4 kpre[4], vpre[4];  // vector values: they stay in VGPRs
    auto slot_key = [&](int i) { return 16 * ((4 * wave + i) & 3) + (lane & 15); };
    auto slot_d4 = [&](int i) { return 4 * ((4 * wave + i) >> 2) + (lane >> 4); };
    // Byte offsets of the slots from the tile's first key row. Each tile is
    // read through a buffer resource (wave-uniform base and size) plus these
    // 32-bit lane offsets, so no per-tile address arithmetic runs on the
    // VALU. The resource ends at this (row, head)'s last key: slots past n_k
    // (a ragged last tile) read as zeros, and the mask discards their scores.
    uint32_t kofs[4], vofs[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        kofs[i] = (uint32_t)((slot_key(i) * ldk + 4 * slot_d4(i)) * sizeof(float));
        vofs[i] = (uint32_t)((slot_key(i) * ldv + 4 * slot_d4(i)) * sizeof(float));
    }
    const uint32_t kbytes = (uint32_t)(((int64_t)(n_k - 1) * ldk + ATT_D) * sizeof(float));
    const uint32_t vbytes = (uint32_t)(((int64_t)(n_k - 1) * ldv + ATT_D) * sizeof(float));
    auto fetch = [&](int key0) {
        const __amdgpu_buffer_rsrc_t rk =
            att_rsrc(kb + (int64_t)key0 * ldk, kbytes - (uint32_t)(key0 * ldk * sizeof(float)));
        const __amdgpu_buffer_rsrc_t rv =
            att_rsrc(vb + (int64_t)key0 * ldv, vbytes - (uint32_t)(key0 * ldv * sizeof(float)));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            kpre[i] = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(rk, kofs[i], 0, 0));
            vpre[i] = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(rv, vofs[i], 0, 0));
        }
    };
    auto stage = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int key = slot_key(i), d = 4 * slot_d4(i);
            *reinterpret_cast<floatx4 *>(&Ks[buf][key][d]) = kpre[i];
            Vt[buf][d + 0][key] = vpre[i][0];
            Vt[buf][d + 1][key] = vpre[i][1];
            Vt[buf][d + 2][key] = vpre[i][2];
            Vt[buf][d + 3][key] = vpre[i][3];
        }
    };

    const floatx16 zero = {};
    floatx16 o0 = zero, o1 = zero;
    float m_run = -INFINITY, l_run = 0.0f;
    // The score accumulators start at -mb (in every register) instead of 0,
    // so the MFMAs deliver s - mb: mb is the running max once the first tile
    // has set it (0 before), and the common tile needs no subtraction before
    // its exponentials. thr is the rescale threshold on s - mb: -inf until
    // the first tile, then ATT_SLACK.
    floatx16 negmb = zero;
    float mb = 0.0f, thr = -INFINITY;

    // One 64-key tile; MASK only for a ragged last tile.
    auto tile = [&](auto mask_tag, int buf, int key0) {
        constexpr bool MASK = decltype(mask_tag)::value;
        // S^T - mb for keys [key0, key0+32) (s0) and [key0+32, key0+64) (s1).
        floatx16 s0, s1;
        att_prio(1);
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const float4 ka = lds4(&Ks[buf][j][32 * half + 4 * c]);
            const float4 kc = lds4(&Ks[buf][32 + j][32 * half + 4 * c]);
            const float av[4] = {ka.x, ka.y, ka.z, ka.w};
            const float cv[4] = {kc.x, kc.y, kc.z, kc.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int s = 4 * c + e;
                s0 = __builtin_amdgcn_mfma_f32_32x32x2f32(av[e], qreg[s], s == 0 ? negmb : s0, 0, 0, 0);
                s1 = __builtin_amdgcn_mfma_f32_32x32x2f32(cv[e], qreg[s], s == 0 ? negmb : s1, 0, 0, 0);
            }
        }
        // Register r of lane l holds key key0 + 8*(r/4) + 4*half + r%4 (s0), +32 (s1).
        if constexpr (MASK) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int kk = key0 + 8 * (r >> 2) + 4 * half + (r & 3);
                if (kk >= n_k) s0[r] = -INFINITY;
                if (kk + 32 >= n_k) s1[r] = -INFINITY;
            }
        }
        att_prio(0);
        float mloc = fmaxf(s0[0], s1[0]);
#pragma unroll
        for (int r = 1; r < 16; ++r) mloc = fmaxf(mloc, fmaxf(s0[r], s1[r]));
        mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
        if (__any(mloc > thr)) {  // uniform branch; always taken on the first tile
            const float m_new = fmaxf(m_run, mloc + mb);
            const float corr = __builtin_amdgcn_exp2f(m_run - m_new);  // 0 on the first tile: O, l are 0
            const float shift = m_new - mb;
            l_run *= corr;
            m_run = m_new;
            mb = m_new;
            thr = ATT_SLACK;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                o0[r] *= corr;
                o1[r] *= corr;
                s0[r] -= shift;
                s1[r] -= shift;
                negmb[r] = -m_new;
            }
        }
        float lsum = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            s0[r] = __builtin_amdgcn_exp2f(s0[r]);
            s1[r] = __builtin_amdgcn_exp2f(s1[r]);
            lsum += s0[r] + s1[r];
        }
        lsum += __shfl_xor(lsum, 32, 64);
        l_run += lsum;
        att_prio(1);
        // O^T += V^T P^T, contracting keys in the order the score registers
        // hold them: registers 4a..4a+3 are keys 8a + 4*half + 0..3.
#pragma unroll
        for (int a = 0; a < 4; ++a) {
            const float4 v0 = lds4(&Vt[buf][j][8 * a + 4 * half]);
            const float4 v1 = lds4(&Vt[buf][32 + j][8 * a + 4 * half]);
            const float4 w0 = lds4(&Vt[buf][j][32 + 8 * a + 4 * half]);
            const float4 w1 = lds4(&Vt[buf][32 + j][32 + 8 * a + 4 * half]);
            const float v0v[4] = {v0.x, v0.y, v0.z, v0.w}, v1v[4] = {v1.x, v1.y, v1.z, v1.w};
            const float w0v[4] = {w0.x, w0.y, w0.z, w0.w}, w1v[4] = {w1.x, w1.y, w1.z, w1.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                o0 = __builtin_amdgcn_mfma_f32_32x32x2f32(v0v[e], s0[4 * a + e], o0, 0, 0, 0);
                o1 = __builtin_amdgcn_mfma_f32_32x32x2f32(v1v[e], s0[4 * a + e], o1, 0, 0, 0);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                o0 = __builtin_amdgcn_mfma_f32_32x32x2f32(w0v[e], s1[4 * a + e], o0, 0, 0, 0);
                o1 = __builtin_amdgcn_mfma_f32_32x32x2f32(w1v[e], s1[4 * a + e], o1, 0, 0, 0);
            }
        }
        att_prio(0);
    };

    const int tiles = (n_k + ATT_KT - 1) / ATT_KT;
    const bool ragged = (n_k % ATT_KT) != 0;
    // The loop runs the full tiles only; a ragged last tile (the one masked
    // variant) follows it, so the loop body has a single tile variant.
    const int full = tiles - (ragged ? 1 : 0);
    // A wave whose 32 queries all lie past n_q (the back half of a last query
    // block when n_q is an odd multiple of 64) stages its share of every tile
    // and takes part in the barriers, but skips the multiplies: its SIMD's
    // matrix core is left to the other workgroup's wave.
    const bool wave_active =
        qblock * (ATT_QW * ATT_WAVES) + __builtin_amdgcn_readfirstlane(wave) * ATT_QW < n_q;
    fetch(0);
    stage(0);
    __syncthreads();
    for (int t = 0; t < full; ++t) {
        const int buf = t & 1;
        const bool more = t + 1 < tiles;
        // The next tile's loads go out before this tile's MFMAs (on the last
        // tile they fetch it again, unused): unconditional, and pinned ahead
        // of the MFMAs by the scheduling barrier.
        fetch(min(t + 1, tiles - 1) * ATT_KT);
        __builtin_amdgcn_sched_barrier(0);
        if (wave_active) tile(std::false_type{}, buf, t * ATT_KT);
        if (more) {
            // The other buffer was last read in tile t-1, which every wave
            // finished before the previous barrier.
            stage(buf ^ 1);
            __syncthreads();
        }
    }
    if (ragged && wave_active) tile(std::true_type{}, full & 1, full * ATT_KT);

    if (!q_ok) return;
    const float inv = l_run > 0.0f ? 1.0f / l_run : 1.0f;
    // Register r of o0/o1 holds dim (0|32) + 8*(r/4) + 4*half + r%4.
    att_store(P_, b * o_bs + (int64_t)qi * ldo + head * ATT_D, half, o0, o1, inv);
}

// ---------------------------------------------------------------------------
// bf16-MFMA variant: Q, K, V and P enter v_mfma_f32_32x32x16_bf16 rounded to
// bf16; scores, softmax, the running max/sum and O stay fp32. Same layout as
// the fp32 kernel with 16-deep contractions: per 64-key tile, 8 MFMAs for
// S^T = K Q^T and 8 for O^T += V^T P^T. The score registers 8m .. 8m+7 of a
// lane (keys 16m + 8(e/4) + 4*half + e%4) are exactly one bf16x8 B operand, so
// V^T is read as two 4-key runs per operand.
// ---------------------------------------------------------------------------

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float floatx8 __attribute__((ext_vector_type(8)));

constexpr int ATT_LDK16 = 72;  // bf16 per K row (144 B: 16-byte aligned, conflict-free b128 reads)
constexpr int ATT_LDV16 = 68;  // bf16 per V^T row (136 B: conflict-free b64 reads)

__device__ __forceinline__ bf16x8 to_bf16x8(floatx8 v) { return __builtin_convertvector(v, bf16x8); }

__global__ __launch_bounds__(256) void attention_bf16_kernel(const AttGroup g) {
    DMX_ATT_LOCATE(g)
    __shared__ __align__(16) __bf16 Ks[2][ATT_KT][ATT_LDK16];  // [buffer][key][d]
    __shared__ __align__(16) __bf16 Vt[2][ATT_D][ATT_LDV16];   // [buffer][d][key]

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int j = lane & 31, half = lane >> 5;
    const int qi = qblock * (ATT_QW * ATT_WAVES) + wave * ATT_QW + j;
    const bool q_ok = qi < n_q;

    const float *qb = q + b * q_bs + head * ATT_D;
    const float *kb = k + b * kv_bs + head * ATT_D;
    const float *vb = v + b * kv_bs + head * ATT_D;

    // Q fragments: dims 16t + 8*half .. +7, pre-scaled into log2 units.
    bf16x8 qf[4];
    {
        const float qs = scale * ATT_LOG2E;
        const float *row = qb + (int64_t)(q_ok ? qi : 0) * ldq + 8 * half;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            floatx8 x = {};
            if (q_ok) {
                const float4 a = *reinterpret_cast<const float4 *>(row + 16 * t);
                const float4 c = *reinterpret_cast<const float4 *>(row + 16 * t + 4);
                x = (floatx8){a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
            }
            qf[t] = to_bf16x8(x * qs);
        }
    }

    floatx4 kpre[4], vpre[4];
    auto slot_key = [&](int i) { return 16 * ((4 * wave + i) & 3) + (lane & 15); };
    auto slot_d4 = [&](int i) { return 4 * ((4 * wave + i) >> 2) + (lane >> 4); };
    // Tiles are read through buffer resources, as in the fp32 kernel: slots
    // past n_k read as zeros and the mask discards their scores.
    uint32_t kofs[4], vofs[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        kofs[i] = (uint32_t)((slot_key(i) * ldk + 4 * slot_d4(i)) * sizeof(float));
        vofs[i] = (uint32_t)((slot_key(i) * ldv + 4 * slot_d4(i)) * sizeof(float));
    }
    const uint32_t kbytes = (uint32_t)(((int64_t)(n_k - 1) * ldk + ATT_D) * sizeof(float));
    const uint32_t vbytes = (uint32_t)(((int64_t)(n_k - 1) * ldv + ATT_D) * sizeof(float));
    auto fetch = [&](int key0) {
        const __amdgpu_buffer_rsrc_t rk =
            att_rsrc(kb + (int64_t)key0 * ldk, kbytes - (uint32_t)(key0 * ldk * sizeof(float)));
        const __amdgpu_buffer_rsrc_t rv =
            att_rsrc(vb + (int64_t)key0 * ldv, vbytes - (uint32_t)(key0 * ldv * sizeof(float)));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            kpre[i] = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(rk, kofs[i], 0, 0));
            vpre[i] = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(rv, vofs[i], 0, 0));
        }
    };
    auto stage = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int key = slot_key(i), d = 4 * slot_d4(i);
            const bf16x4 kv = __builtin_convertvector(kpre[i], bf16x4);
            *reinterpret_cast<bf16x4 *>(&Ks[buf][key][d]) = kv;
            const bf16x4 vv = __builtin_convertvector(vpre[i], bf16x4);
            Vt[buf][d + 0][key] = vv[0];
            Vt[buf][d + 1][key] = vv[1];
            Vt[buf][d + 2][key] = vv[2];
            Vt[buf][d + 3][key] = vv[3];
        }
    };
    // V^T operand for dim row d and keys base + 8(e/4) + 4*half + e%4.
    auto vfrag = [&](int buf, int d, int base) -> bf16x8 {
        const bf16x4 lo = *reinterpret_cast<const bf16x4 *>(&Vt[buf][d][base + 4 * half]);
        const bf16x4 hi = *reinterpret_cast<const bf16x4 *>(&Vt[buf][d][base + 8 + 4 * half]);
        return (bf16x8){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    };

    const floatx16 zero = {};
    floatx16 o0 = zero, o1 = zero;
    float m_run = -INFINITY, l_run = 0.0f;
    // Scores accumulate onto -mb, as in the fp32 kernel.
    floatx16 negmb = zero;
    float mb = 0.0f, thr = -INFINITY;

    auto tile = [&](auto mask_tag, int buf, int key0) {
        constexpr bool MASK = decltype(mask_tag)::value;
        floatx16 s0 = negmb, s1 = negmb;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const bf16x8 ka = *reinterpret_cast<const bf16x8 *>(&Ks[buf][j][16 * t + 8 * half]);
            const bf16x8 kc = *reinterpret_cast<const bf16x8 *>(&Ks[buf][32 + j][16 * t + 8 * half]);
            s0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka, qf[t], s0, 0, 0, 0);
            s1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kc, qf[t], s1, 0, 0, 0);
        }
        if constexpr (MASK) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int kk = key0 + 8 * (r >> 2) + 4 * half + (r & 3);
                if (kk >= n_k) s0[r] = -INFINITY;
                if (kk + 32 >= n_k) s1[r] = -INFINITY;
            }
        }
        float mloc = fmaxf(s0[0], s1[0]);
#pragma unroll
        for (int r = 1; r < 16; ++r) mloc = fmaxf(mloc, fmaxf(s0[r], s1[r]));
        mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
        if (__any(mloc > thr)) {
            const float m_new = fmaxf(m_run, mloc + mb);
            const float corr = __builtin_amdgcn_exp2f(m_run - m_new);
            const float shift = m_new - mb;
            l_run *= corr;
            m_run = m_new;
            mb = m_new;
            thr = ATT_SLACK;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                o0[r] *= corr;
                o1[r] *= corr;
                s0[r] -= shift;
                s1[r] -= shift;
                negmb[r] = -m_new;
            }
        }
        float lsum = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            s0[r] = __builtin_amdgcn_exp2f(s0[r]);
            s1[r] = __builtin_amdgcn_exp2f(s1[r]);
            lsum += s0[r] + s1[r];
        }
        lsum += __shfl_xor(lsum, 32, 64);
        l_run += lsum;
#pragma unroll
        for (int m = 0; m < 2; ++m) {
            const bf16x8 p0 = to_bf16x8((floatx8){s0[8 * m], s0[8 * m + 1], s0[8 * m + 2], s0[8 * m + 3],
                                                  s0[8 * m + 4], s0[8 * m + 5], s0[8 * m + 6], s0[8 * m + 7]});
            const bf16x8 p1 = to_bf16x8((floatx8){s1[8 * m], s1[8 * m + 1], s1[8 * m + 2], s1[8 * m + 3],
                                                  s1[8 * m + 4], s1[8 * m + 5], s1[8 * m + 6], s1[8 * m + 7]});
            o0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vfrag(buf, j, 16 * m), p0, o0, 0, 0, 0);
            o1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vfrag(buf, 32 + j, 16 * m), p0, o1, 0, 0, 0);
            o0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vfrag(buf, j, 32 + 16 * m), p1, o0, 0, 0, 0);
            o1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vfrag(buf, 32 + j, 32 + 16 * m), p1, o1, 0, 0, 0);
        }
    };

    const int tiles = (n_k + ATT_KT - 1) / ATT_KT;
    const bool ragged = (n_k % ATT_KT) != 0;
    const int full = tiles - (ragged ? 1 : 0);
    const bool wave_active =
        qblock * (ATT_QW * ATT_WAVES) + __builtin_amdgcn_readfirstlane(wave) * ATT_QW < n_q;
    fetch(0);
    stage(0);
    __syncthreads();
    for (int t = 0; t < full; ++t) {
        const int buf = t & 1;
        const bool more = t + 1 < tiles;
        fetch(min(t + 1, tiles - 1) * ATT_KT);
        __builtin_amdgcn_sched_barrier(0);
        if (wave_active) tile(std::false_type{}, buf, t * ATT_KT);
        if (more) {
            stage(buf ^ 1);
            __syncthreads();
        }
    }
    if (ragged && wave_active) tile(std::true_type{}, full & 1, full * ATT_KT);

    if (!q_ok) return;
    const float inv = l_run > 0.0f ? 1.0f / l_run : 1.0f;
    // Register r of o0/o1 holds dim (0|32) + 8*(r/4) + 4*half + r%4.
    att_store(P_, b * o_bs + (int64_t)qi * ldo + head * ATT_D, half, o0, o1, inv);
}

// ---------------------------------------------------------------------------
// Three-plane variant: fp32 accuracy on the bf16 matrix cores. Q, K, V and
// the probabilities P are each held as three bf16 planes (x = x0 + x1 + x2,
// every fp32 value exactly), and each product sums the six plane products
// a_i b_j with i + j < 3 on v_mfma_f32_32x32x16_bf16; the dropped ones are
// below 2^-24 of |a b|. Scores, softmax, running max/sum and O stay fp32 as
// in the fp32 kernel, with the same transposed layout (S^T = K Q^T, then
// O^T += V^T P^T with P straight from the score registers).
// K and V arrive as planes (KVPlanes: the in-projection's epilogue writes
// them, once per token, instead of every query block splitting its tiles):
// K [token][d], V^T [d][token] with each 16-token group in the order 0-3,
// 8-11, 4-7, 12-15, which is the key order of a lane's B operand, so every
// operand is one 16-byte LDS read and staging is plain 16-byte copies.
// Key tiles are 32 keys, double buffered: the three planes of a K tile and a
// V^T tile take 54 KB, so two workgroups (two waves per SIMD) share a CU.
// Software pipeline: while a wave turns tile t's scores into probabilities
// (exponentials, row sums, plane splits: VALU work) it issues the 24 score
// MFMAs of tile t + 1 between those instructions, so the VALU work runs in
// the matrix core's busy cycles; then come tile t's 24 P V MFMAs. The K
// buffers run one tile ahead of the V^T buffers, and one barrier per tile
// covers both.
// ---------------------------------------------------------------------------

constexpr int AX_KT = 32;   // keys per tile
constexpr int AX_LDK = 72;  // bf16 per K row (144 B: conflict-free b128 reads)
constexpr int AX_LDV = 40;  // bf16 per V^T row (80 B: conflict-free b128 reads)

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// max / sum of x over a lane pair (l, l + 32), one v_permlane32_swap: the
// swap leaves the lower lane's value in one register and the upper lane's
// in the other on both lanes, so both get the same bits. Inline asm: the
// compiler's builtin for this instruction returned the first register for
// both results. The nops cover the VALU-write -> permlane-read and
// permlane-write -> VALU-read dependencies.
__device__ __forceinline__ void att_swap_halves(float x, float &a, float &b) {
    unsigned u = __builtin_bit_cast(unsigned, x), w = u;
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(u), "+v"(w));
    a = __builtin_bit_cast(float, u);
    b = __builtin_bit_cast(float, w);
}
__device__ __forceinline__ float att_pair_max(float x) {
    float a, b;
    att_swap_halves(x, a, b);
    return fmaxf(a, b);
}
__device__ __forceinline__ float att_pair_sum(float x) {
    float a, b;
    att_swap_halves(x, a, b);
    return a + b;
}

// Three bf16 planes of fp32 values, round to nearest even at each step:
// a plane pair h = (bf16(x0), bf16(x1)) is one v_cvt_pk_bf16_f32, and the
// residuals x - plane (exact in fp32) take the planes' bits straight from
// the packed pair (low half << 16, high half & 0xffff0000).
__device__ __forceinline__ void att_residual(bf16x2 h, float &x0, float &x1) {
    const unsigned u = __builtin_bit_cast(unsigned, h);
    x0 -= __builtin_bit_cast(float, u << 16);
    x1 -= __builtin_bit_cast(float, u & 0xffff0000u);
}

__device__ __forceinline__ void split3(floatx8 x, bf16x8 &p0, bf16x8 &p1, bf16x8 &p2) {
    auto step = [](floatx8 &v) {
        const bf16x8 h = __builtin_convertvector(v, bf16x8);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float x0 = v[2 * e], x1 = v[2 * e + 1];
            att_residual((bf16x2){h[2 * e], h[2 * e + 1]}, x0, x1);
            v[2 * e] = x0;
            v[2 * e + 1] = x1;
        }
        return h;
    };
    p0 = step(x);
    p1 = step(x);
    p2 = __builtin_convertvector(x, bf16x8);
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void attention_x3_kernel(const AttGroup g) {
    DMX_ATT_LOCATE(g)
    __shared__ __align__(16) __bf16 Ks[2][3][AX_KT][AX_LDK];  // [buffer][plane][key][d]
    __shared__ __align__(16) __bf16 Vt[2][3][ATT_D][AX_LDV];  // [buffer][plane][d][key, permuted]
    (void)k;
    (void)v;
    (void)ldk;
    (void)ldv;
    (void)kv_bs;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int j = lane & 31, half = lane >> 5;
    const int qi = qblock * (ATT_QW * ATT_WAVES) + wave * ATT_QW + j;
    const bool q_ok = qi < n_q;
    const float *qb = q + b * q_bs + head * ATT_D;

    // Q planes: dims 16t + 8*half .. +7, pre-scaled into log2 units.
    bf16x8 qf[3][4];
    {
        const float qs = scale * ATT_LOG2E;
        const float *row = qb + (int64_t)(q_ok ? qi : 0) * ldq + 8 * half;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            floatx8 x = {};
            if (q_ok) {
                const float4 a = *reinterpret_cast<const float4 *>(row + 16 * t);
                const float4 c = *reinterpret_cast<const float4 *>(row + 16 * t + 4);
                x = (floatx8){a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
            }
            split3(x * qs, qf[0][t], qf[1][t], qf[2][t]);
        }
    }

    // Staging: 16-byte chunk slot tid of every plane. K: key tid / 8, dims
    // 8 (tid % 8) .. +7; V^T: dim tid / 4, stored keys 8 (tid % 4) .. +7.
    // K rows are read through a buffer resource that ends at this (row,
    // head)'s last key, so a ragged last tile reads zeros past it; V^T rows
    // are zero from n_k to ldvt.
    const unsigned short *kpb = P_.kp + b * P_.kp_bs + head * ATT_D;
    const unsigned short *vtb = P_.vt + ((int64_t)b * P_.heads + head) * ATT_D * P_.ldvt;
    const int64_t kld = P_.kp_ld;
    const uint32_t kofs = (uint32_t)(((tid >> 3) * kld + 8 * (tid & 7)) * sizeof(unsigned short));
    const uint32_t vofs = (uint32_t)(((tid >> 2) * P_.ldvt + 8 * (tid & 3)) * sizeof(unsigned short));
    const uint32_t kbytes = (uint32_t)(((int64_t)(n_k - 1) * kld + ATT_D) * sizeof(unsigned short));
    floatx4 kpre[3], vpre[3];
    auto fetch_k = [&](int key0) {
#pragma unroll
        for (int pl = 0; pl < 3; ++pl) {
            const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<unsigned short *>(kpb + pl * P_.kp_ps + (int64_t)key0 * kld), (short)0,
                (int)(kbytes - (uint32_t)(key0 * kld * sizeof(unsigned short))), 0x00020000);
            kpre[pl] = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(rk, kofs, 0, 0));
        }
    };
    auto fetch_v = [&](int key0) {
#pragma unroll
        for (int pl = 0; pl < 3; ++pl)
            vpre[pl] = *reinterpret_cast<const floatx4 *>(reinterpret_cast<const char *>(vtb + pl * P_.vt_ps + key0) +
                                                          vofs);
    };
    auto stage_k = [&](int buf) {
#pragma unroll
        for (int pl = 0; pl < 3; ++pl)
            *reinterpret_cast<floatx4 *>(&Ks[buf][pl][tid >> 3][8 * (tid & 7)]) = kpre[pl];
    };
    auto stage_v = [&](int buf) {
#pragma unroll
        for (int pl = 0; pl < 3; ++pl)
            *reinterpret_cast<floatx4 *>(&Vt[buf][pl][tid >> 2][8 * (tid & 3)]) = vpre[pl];
    };

    // Scores stay raw (log2 units); mb is the offset of the exponentials,
    // exp2(s - mb), raised lazily: only when some query's tile max exceeds
    // lim = mb + ATT_SLACK (always on the first tile, lim = -inf).
    const floatx16 zero = {};
    floatx16 o0 = zero, o1 = zero;
    float mb = -INFINITY, lim = -INFINITY, l_run = 0.0f;

    // Score MFMA i of k-group t4 of the tile whose K fragments are kf, onto
    // acc; smallest products first.
    auto score_mfma = [&](int t4, int i, const bf16x8 (&kf)[3], floatx16 acc) {
        constexpr int ka[6] = {2, 1, 0, 1, 0, 0}, qa[6] = {0, 1, 2, 0, 1, 0};
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[ka[i]], qf[qa[i]][t4], acc, 0, 0, 0);
    };
    auto read_k = [&](int buf, int t4, bf16x8 (&kf)[3]) {
#pragma unroll
        for (int pl = 0; pl < 3; ++pl) kf[pl] = *reinterpret_cast<const bf16x8 *>(&Ks[buf][pl][j][16 * t4 + 8 * half]);
    };
    // Scores of the tile in K buffer buf: register r holds key 8(r/4) +
    // 4*half + r%4 of the tile.
    auto scores = [&](int buf) {
        floatx16 sc = zero;
#pragma unroll
        for (int t4 = 0; t4 < 4; ++t4) {
            bf16x8 kf[3];
            read_k(buf, t4, kf);
#pragma unroll
            for (int i = 0; i < 6; ++i) sc = score_mfma(t4, i, kf, sc);
        }
        return sc;
    };
    auto row_max = [&](const floatx16 &sc) {
        float mloc = sc[0];
#pragma unroll
        for (int r = 1; r < 16; ++r) mloc = fmaxf(mloc, sc[r]);
        return att_pair_max(mloc);
    };
    // Raises mb to the running max when some query's tile max mloc exceeds
    // lim, rescaling O and the row sum (O and the sum carry the same factor,
    // which the final division cancels).
    auto raise_max = [&](float mloc) {
        if (__any(mloc > lim)) {
            const float m_new = fmaxf(mb, mloc);
            const float corr = __builtin_amdgcn_exp2f(mb - m_new);
            l_run *= corr;
            mb = m_new;
            lim = m_new + ATT_SLACK;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                o0[r] *= corr;
                o1[r] *= corr;
            }
        }
    };
    // P's planes in the B-operand order: registers 8m .. 8m+7 are keys
    // 16m + 4*half + 0..3 and 16m + 8 + 4*half + 0..3, which V^T stores
    // contiguously at 16m + 8*half. Plane word pw[q][m][e] holds registers
    // 8m + 2e and 8m + 2e + 1.
    typedef unsigned uintx4 __attribute__((ext_vector_type(4)));
    auto split_pair = [&](const floatx16 &p, int u, uintx4 (&pw)[3][2]) {
        const int m = u / 4, e = u % 4;
        float x0 = p[2 * u], x1 = p[2 * u + 1];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const bf16x2 h = {(__bf16)x0, (__bf16)x1};
            pw[q][m][e] = __builtin_bit_cast(unsigned, h);
            att_residual(h, x0, x1);
        }
        const bf16x2 h = {(__bf16)x0, (__bf16)x1};
        pw[2][m][e] = __builtin_bit_cast(unsigned, h);
    };
    auto planes_of = [&](const uintx4 (&pw)[3][2], bf16x8 (&pp)[3][2]) {
#pragma unroll
        for (int q = 0; q < 3; ++q)
#pragma unroll
            for (int m = 0; m < 2; ++m) pp[q][m] = __builtin_bit_cast(bf16x8, pw[q][m]);
    };
    auto read_v = [&](int buf, int m, bf16x8 (&va)[3], bf16x8 (&vc)[3]) {
#pragma unroll
        for (int pl = 0; pl < 3; ++pl) {
            va[pl] = *reinterpret_cast<const bf16x8 *>(&Vt[buf][pl][j][16 * m + 8 * half]);
            vc[pl] = *reinterpret_cast<const bf16x8 *>(&Vt[buf][pl][32 + j][16 * m + 8 * half]);
        }
    };
    // P V MFMA i (0..11) of key half m: o0 for dims 0-31, o1 for 32-63,
    // smallest products first.
    auto pv_mfma = [&](int m, int i, const bf16x8 (&va)[3], const bf16x8 (&vc)[3], const bf16x8 (&pp)[3][2]) {
        constexpr int vp[6] = {2, 1, 0, 1, 0, 0}, ppl[6] = {0, 1, 2, 0, 1, 0};
        if (i % 2 == 0)
            o0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va[vp[i / 2]], pp[ppl[i / 2]][m], o0, 0, 0, 0);
        else
            o1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vc[vp[i / 2]], pp[ppl[i / 2]][m], o1, 0, 0, 0);
    };

    const int tiles = (n_k + AX_KT - 1) / AX_KT;
    const bool ragged = (n_k % AX_KT) != 0;
    const bool wave_active =
        qblock * (ATT_QW * ATT_WAVES) + __builtin_amdgcn_readfirstlane(wave) * ATT_QW < n_q;

    // Tile t of the pipelined run (t + 1 < tiles). cur holds tile t's raw
    // scores and mrow their row max; nxt and mrow receive tile t + 1's.
    // Scheduling fences fix the instruction order: each of the 24 score
    // MFMAs of tile t + 1 is followed by a share of tile t's softmax (one
    // exponential and one row-sum add on each of the first 16, then the
    // plane splits of one key pair each), each k-group's K reads go out a
    // k-group ahead, and the first key half's V^T fragments during the last
    // score MFMAs (the second half's after the first P V MFMA); the row max
    // of tile t + 1 runs between tile t's P V MFMAs. Then the staging of K
    // tile t + 2 and V^T tile t + 1: K buffer t & 1 last held tile t and V^T
    // buffer (t + 1) & 1 tile t - 1, both read before the last barrier.
    auto pipelined = [&](int t, floatx16 &cur, floatx16 &nxt, float &mrow) {
        if (t + 2 < tiles) fetch_k((t + 2) * AX_KT);
        fetch_v((t + 1) * AX_KT);
        __builtin_amdgcn_sched_barrier(0);
        if (wave_active) {
            raise_max(mrow);
            const int kb = (t + 1) & 1, vb = t & 1;
            float lsum = 0.0f;
            uintx4 pw[3][2];
            bf16x8 kf[2][3];
            bf16x8 va[2][3], vc[2][3];
            floatx16 acc = zero;
            read_k(kb, 0, kf[0]);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int s = 0; s < 24; ++s) {
                const int t4 = s / 6, i = s % 6;
                acc = score_mfma(t4, i, kf[t4 & 1], acc);
                if (i == 0 && t4 < 3) read_k(kb, t4 + 1, kf[(t4 + 1) & 1]);
                // V^T fragments of the first key half, ahead of the P V MFMAs.
                if (s == 19) read_v(vb, 0, va[0], vc[0]);
                if (s < 16) cur[s] = __builtin_amdgcn_exp2f(cur[s] - mb);
                if (s >= 1 && s <= 16) lsum += cur[s - 1];
                if (s >= 16) split_pair(cur, s - 16, pw);
                if (s == 23) l_run += att_pair_sum(lsum);
                __builtin_amdgcn_sched_barrier(0);
            }
            nxt = acc;
            bf16x8 pp[3][2];
            planes_of(pw, pp);
            float mx = 0.0f;
#pragma unroll
            for (int m = 0; m < 2; ++m) {
#pragma unroll
                for (int i = 0; i < 12; ++i) {
                    pv_mfma(m, i, va[m], vc[m], pp);
                    // The second key half's fragments after the first MFMA.
                    if (m == 0 && i == 0) read_v(vb, 1, va[1], vc[1]);
                    const int s = 12 * m + i;
                    if (s == 2) mx = fmaxf(nxt[0], nxt[1]);
                    if (s >= 3 && s <= 9) mx = fmaxf(fmaxf(mx, nxt[2 * s - 4]), nxt[2 * s - 3]);
                    if (s == 10) mrow = att_pair_max(mx);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        if (t + 2 < tiles) stage_k(t & 1);
        stage_v((t + 1) & 1);
        __syncthreads();
    };
    // The last tile (masked past n_k when ragged), not overlapped.
    auto last = [&](int t, floatx16 &cur) {
        if (!wave_active) return;
        if (ragged) {
#pragma unroll
            for (int r = 0; r < 16; ++r)
                if (t * AX_KT + 8 * (r >> 2) + 4 * half + (r & 3) >= n_k) cur[r] = -INFINITY;
        }
        raise_max(row_max(cur));
        float lsum = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            cur[r] = __builtin_amdgcn_exp2f(cur[r] - mb);
            lsum += cur[r];
        }
        l_run += att_pair_sum(lsum);
        uintx4 pw[3][2];
#pragma unroll
        for (int u = 0; u < 8; ++u) split_pair(cur, u, pw);
        bf16x8 pp[3][2];
        planes_of(pw, pp);
#pragma unroll
        for (int m = 0; m < 2; ++m) {
            bf16x8 va[3], vc[3];
            read_v(t & 1, m, va, vc);
#pragma unroll
            for (int i = 0; i < 12; ++i) pv_mfma(m, i, va, vc, pp);
        }
    };

    // Prologue: K and V^T of tile 0 and K of tile 1 staged; tile 0's scores.
    // The second barrier: K buffer 0 takes tile 2 at the end of the first
    // tile, after every wave has read tile 0 from it.
    fetch_k(0);
    fetch_v(0);
    stage_k(0);
    stage_v(0);
    if (tiles > 1) {
        fetch_k(AX_KT);
        stage_k(1);
    }
    __syncthreads();
    floatx16 sa = zero, sb = zero;
    float mrow = 0.0f;
    if (wave_active) {
        sa = scores(0);
        mrow = row_max(sa);
    }
    __syncthreads();
    // Two tiles per trip, so the two score registers swap roles without
    // copies.
    int t = 0;
    for (; t + 2 < tiles; t += 2) {
        pipelined(t, sa, sb, mrow);
        pipelined(t + 1, sb, sa, mrow);
    }
    if (t + 1 < tiles) {
        pipelined(t, sa, sb, mrow);
        last(t + 1, sb);
    } else {
        last(t, sa);
    }

    if (!q_ok) return;
    const float inv = l_run > 0.0f ? 1.0f / l_run : 1.0f;
    att_store(P_, b * o_bs + (int64_t)qi * ldo + head * ATT_D, half, o0, o1, inv);
}

// fp32 K rows -> K planes, four dims per thread.
__global__ __launch_bounds__(256) void k_planes_kernel(const float *__restrict__ k, int64_t ldk, int64_t kv_bs,
                                                       int n_k, int D, unsigned short *__restrict__ out,
                                                       int64_t stride, int64_t bs, int64_t ld) {
    const int b = blockIdx.y;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // (token, dim quad)
    const int quads = D / 4;
    if (i >= (int64_t)n_k * quads) return;
    const int64_t t = i / quads;
    const int d = 4 * (int)(i % quads);
    const float4 x = *reinterpret_cast<const float4 *>(k + b * kv_bs + t * ldk + d);
    store_planes4<3>(out + b * bs + t * ld + d, stride, x);
}

// fp32 V rows -> V^T planes, four stored tokens of one dim per thread (zeros
// past n_k).
__global__ __launch_bounds__(256) void vt_planes_kernel(const float *__restrict__ v, int64_t ldv, int64_t kv_bs,
                                                        int n_k, int D, int64_t ldvt,
                                                        unsigned short *__restrict__ out, int64_t stride) {
    const int b = blockIdx.y;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // (column, stored-token quad)
    const int64_t quads = ldvt / 4;
    if (i >= (int64_t)D * quads) return;
    const int col = (int)(i % D);
    const int64_t pos = 4 * (i / D);
    float x[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int64_t t = vt_token_pos(pos + e);  // the permutation is its own inverse
        x[e] = t < n_k ? v[b * kv_bs + t * ldv + col] : 0.0f;
    }
    // Row (b * heads + h) * 64 + d is b * D + col.
    store_planes4<3>(out + ((int64_t)b * D + col) * ldvt + pos, stride, make_float4(x[0], x[1], x[2], x[3]));
}

}  // namespace

// The three-plane kernel serves the fp32 precision unless DMX_ATT_PLANES=0
// (read once) keeps the fp32-MFMA kernel there.
bool attention_planes_enabled() {
    static const bool on = [] {
        const char *e = std::getenv("DMX_ATT_PLANES");
        return !e || std::atoi(e) != 0;
    }();
    return on;
}

void attention_grouped(hipStream_t s, const AttentionArgs *probs, int count, float scale) {
    DMX_REQUIRE(count >= 1 && count <= 2, "attention: one or two problems per launch");
    AttGroup g{};
    g.count = count;
    g.scale = scale;
    int64_t total = 0;
    // Longer blocks (more keys) first: the tail of the launch is then made of
    // the short ones.
    int order[2] = {0, 1};
    if (count == 2 && probs[1].n_k > probs[0].n_k) std::swap(order[0], order[1]);
    const bool planes = probs[0].kv.k != nullptr;
    for (int i = 0; i < count; ++i) {
        const AttentionArgs &a = probs[order[i]];
        DMX_REQUIRE((a.kv.k != nullptr) == planes, "attention: both problems of a launch take K/V planes or neither");
        require_ptrs({a.q, a.out_planes.p ? (const void *)a.out_planes.p : (const void *)a.out}, "attention");
        DMX_REQUIRE(!a.out_planes.p || ((a.out_planes.count == 1 || a.out_planes.count == 3) &&
                                        (reinterpret_cast<uintptr_t>(a.out_planes.p) & 7) == 0 &&
                                        a.out_planes.stride % 4 == 0),
                    "attention: output planes must be 1 or 3, 8-byte aligned");
        DMX_REQUIRE(a.d_head == ATT_D, "attention: only d_head = 64 is implemented");
        DMX_REQUIRE(a.n_q > 0 && a.n_k > 0 && a.batch > 0 && a.heads > 0, "attention: empty problem");
        DMX_REQUIRE(a.ldq % 4 == 0 && a.ldo % 4 == 0 && a.q_batch_stride % 4 == 0 && a.out_batch_stride % 4 == 0,
                    "attention: row strides must be multiples of 4 floats");
        DMX_REQUIRE(((reinterpret_cast<uintptr_t>(a.q) |
                      reinterpret_cast<uintptr_t>(a.out_planes.p ? nullptr : a.out)) & 15) == 0,
                    "attention: operands must be 16-byte aligned");
        if (planes) {
            // K tiles are read through buffer resources that end at a (row,
            // head)'s last key; V^T rows hold whole 32-key tiles.
            const KVPlanes &kv = a.kv;
            require_ptrs({kv.k, kv.vt}, "attention planes");
            DMX_REQUIRE(kv.ldk >= (int64_t)a.heads * ATT_D && kv.ldvt >= kv_ldvt(a.n_k) && kv.ldvt % 32 == 0,
                        "attention: K/V planes rows too short");
            DMX_REQUIRE(((reinterpret_cast<uintptr_t>(kv.k) | reinterpret_cast<uintptr_t>(kv.vt)) & 15) == 0 &&
                            kv.k_stride % 8 == 0 && kv.k_bs % 8 == 0 && kv.ldk % 8 == 0 && kv.vt_stride % 8 == 0,
                        "attention: K/V planes must be 16-byte aligned");
            DMX_REQUIRE(((int64_t)(a.n_k - 1) * kv.ldk + ATT_D) * 2 < (1ll << 31),
                        "attention: K extent of one (row, head) exceeds 2 GiB");
        } else {
            require_ptrs({a.k, a.v}, "attention");
            // K/V tiles are read through buffer resources that end at a (row,
            // head)'s last key: rows must not overlap, and the extent must fit
            // the resource's 31-bit size.
            DMX_REQUIRE(a.ldk >= ATT_D && a.ldv >= ATT_D, "attention: K/V rows shorter than d_head");
            DMX_REQUIRE(((int64_t)(a.n_k - 1) * std::max(a.ldk, a.ldv) + ATT_D) * (int64_t)sizeof(float) < (1ll << 31),
                        "attention: K/V extent of one (row, head) exceeds 2 GiB");
            DMX_REQUIRE(a.ldk % 4 == 0 && a.ldv % 4 == 0 && a.kv_batch_stride % 4 == 0,
                        "attention: row strides must be multiples of 4 floats");
            DMX_REQUIRE(((reinterpret_cast<uintptr_t>(a.k) | reinterpret_cast<uintptr_t>(a.v)) & 15) == 0,
                        "attention: operands must be 16-byte aligned");
        }
        AttProblem &p = g.p[i];
        p.q = a.q;
        p.k = a.k;
        p.v = a.v;
        p.out = a.out;
        p.out_planes = a.out_planes.p;
        p.plane_stride = a.out_planes.stride;
        p.planes = a.out_planes.count;
        p.kp = a.kv.k;
        p.vt = a.kv.vt;
        p.kp_ps = a.kv.k_stride;
        p.kp_bs = a.kv.k_bs;
        p.kp_ld = a.kv.ldk;
        p.vt_ps = a.kv.vt_stride;
        p.ldvt = a.kv.ldvt;
        p.ldq = a.ldq;
        p.ldk = a.ldk;
        p.ldv = a.ldv;
        p.ldo = a.ldo;
        p.q_bs = a.q_batch_stride;
        p.kv_bs = a.kv_batch_stride;
        p.o_bs = a.out_batch_stride;
        p.n_q = a.n_q;
        p.n_k = a.n_k;
        p.heads = a.heads;
        p.qblocks = (int)ceil_div(a.n_q, ATT_QW * ATT_WAVES);
        const int64_t blocks = (int64_t)p.qblocks * a.heads * a.batch;
        DMX_REQUIRE(blocks < (1 << 30), "attention: grid too large");
        p.blocks = (int)blocks;
        total += blocks;
    }
    DMX_REQUIRE(total < (1ll << 31), "attention: grid too large");
    const dim3 grid((unsigned)total);
    if (planes)
        hipLaunchKernelGGL(attention_x3_kernel, grid, dim3(256), 0, s, g);
    else if (bf16_mfma())
        hipLaunchKernelGGL(attention_bf16_kernel, grid, dim3(256), 0, s, g);
    else
        hipLaunchKernelGGL(attention_kernel, grid, dim3(256), 0, s, g);
    DMX_LAUNCH_CHECK();
}

void kv_to_planes(hipStream_t s, const float *k, int64_t ldk, const float *v, int64_t ldv, int64_t kv_bs, int batch,
                  int heads, int n_k, const KVPlanes &out) {
    require_ptrs({k, v, out.k, out.vt}, "kv_to_planes");
    const int D = heads * ATT_D;
    DMX_REQUIRE(batch > 0 && n_k > 0 && batch <= 65535, "kv_to_planes: empty or too many batches");
    DMX_REQUIRE(ldk % 4 == 0 && kv_bs % 4 == 0 && (reinterpret_cast<uintptr_t>(k) & 15) == 0,
                "kv_to_planes: K rows must be float4 aligned");
    DMX_REQUIRE(out.ldk >= D && out.ldvt >= kv_ldvt(n_k) && out.ldvt % 32 == 0 && out.k_stride % 4 == 0 &&
                    out.k_bs % 4 == 0 && out.ldk % 4 == 0 && out.vt_stride % 4 == 0 &&
                    ((reinterpret_cast<uintptr_t>(out.k) | reinterpret_cast<uintptr_t>(out.vt)) & 7) == 0,
                "kv_to_planes: output layout");
    const int64_t kq = (int64_t)n_k * (D / 4), vq = (int64_t)D * (out.ldvt / 4);
    hipLaunchKernelGGL(k_planes_kernel, dim3((unsigned)ceil_div(kq, (int64_t)256), (unsigned)batch), dim3(256), 0, s,
                       k, ldk, kv_bs, n_k, D, out.k, out.k_stride, out.k_bs, out.ldk);
    DMX_LAUNCH_CHECK();
    hipLaunchKernelGGL(vt_planes_kernel, dim3((unsigned)ceil_div(vq, (int64_t)256), (unsigned)batch), dim3(256), 0, s,
                       v, ldv, kv_bs, n_k, D, out.ldvt, out.vt, out.vt_stride);
    DMX_LAUNCH_CHECK();
}

void attention(hipStream_t s, const float *q, int64_t ldq, const float *k, int64_t ldk, const float *v, int64_t ldv,
               float *out, int64_t ldo, int batch, int heads, int n_q, int n_k, int d_head, float scale,
               int64_t q_batch_stride, int64_t kv_batch_stride, int64_t out_batch_stride) {
    const AttentionArgs a{q,     ldq,   k,   ldk,    v,        ldv,           out,           ldo,
                          batch, heads, n_q, n_k,    d_head,   q_batch_stride, kv_batch_stride, out_batch_stride};
    attention_grouped(s, &a, 1, scale);
}

}  // namespace dmx
