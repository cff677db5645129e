// gemm.h — the fp32 MFMA GEMM template every contraction of the forward runs on.
//
//   C[z][m][n] = sum_k A[z][m][k] * B[z][k][n]
//
// A and B are not tensors but *loaders*: small functors that fetch one element
// (or four consecutive k) of the logical operand from wherever it lives. That
// is how one kernel serves the linear layers (A = activations, B = W^T), the
// implicit-GEMM convolutions (B = the im2col patch matrix, gathered on the fly
// with zero padding — nothing is materialised), the transposed convolutions
// (one GEMM per output phase), and the DConv branches (B = GroupNorm+GELU of
// the previous conv applied while loading). The epilogue functor receives each
// result element and does the fused tail: bias, GELU, GLU, LayerScale +
// residual, GroupNorm statistics.
//
// CDNA4 mapping: 256 threads = 4 wave64s; each wave owns a (BM/WAVES_M) x
// (BN/WAVES_N) sub-tile computed as 32x32 tiles with v_mfma_f32_32x32x2f32
// (A: lane l holds A[l%32][l/32]; B: lane l holds B[l/32][l%32];
// D: 16 regs, reg r of lane l is D[8*(r/4) + 4*(l/32) + r%4][l%32]).
// Both operand tiles sit in LDS k-contiguous, [row][k], rows padded to BK + 4
// floats so that 16 consecutive rows start on distinct bank quads. The k
// contraction is reordered in groups of 8: at MFMA step t lane half h
// contributes k = 8g + 4h + t, so one ds_read_b128 of row[8g + 4h .. +3]
// feeds four MFMAs. Tiles go global -> registers -> LDS (double buffered, one
// barrier per BK step), so the next tile's global loads overlap this tile's
// MFMAs. k-major sources are read as float4 along k; m/n-major sources are
// read four k at a time per column (coalesced across lanes along m/n).
//
// GLU mode: each wave's m-tiles hold WTM/2 value channels c followed by the
// gate channels C + c of the same outputs (two tiles = 32 channels, or three
// tiles = 48 channels, which fits C = 48 and 96 without padding). A value
// row's gate row is WTM/2 rows further on, which is a multiple of 8, so it
// lies in the same lane: GLU happens in registers and the 2C-channel product
// is never written.
#pragma once

#include <type_traits>

#include "common.h"

namespace dmx {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// LLVM AMDGPU scheduling strategy for the k-loop (iglp_opt).
#ifndef DMX_GEMM_IGLP
#define DMX_GEMM_IGLP 1
#endif

// k-tile depth of the fp32 kernel (the bf16 kernel stages 32).
#ifndef DMX_GEMM_BK
#define DMX_GEMM_BK 16
#endif
constexpr int GEMM_BK = DMX_GEMM_BK;
constexpr int GEMM_THREADS = 256;

// Round-to-nearest-even fp32 -> bf16 of four values (two v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint2 pack_bf16x4(float4 v) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    const b2 lo = __builtin_convertvector((f2){v.x, v.y}, b2);
    const b2 hi = __builtin_convertvector((f2){v.z, v.w}, b2);
    return make_uint2(__builtin_bit_cast(unsigned, lo), __builtin_bit_cast(unsigned, hi));
}

// Stage element type and depth: fp32 stages BK = 16 floats per row; bf16
// stages 32 (one v_mfma_f32_32x32x16_bf16 per 16, operands 8 bf16 per lane).
template <bool BF16>
struct GemmStage {
    using T = float;
    static constexpr int BK = GEMM_BK;
};
template <>
struct GemmStage<true> {
    using T = unsigned short;
    static constexpr int BK = 32;
};

template <int BM, int BN, int WAVES_M, bool GLU, bool BF16, class AL, class BL, class EP>
__global__ __launch_bounds__(GEMM_THREADS) void gemm_kernel(int M, int N, int K, AL al, BL bl, EP ep) {
    using T = typename GemmStage<BF16>::T;
    constexpr int BK = GemmStage<BF16>::BK;
    constexpr int KQ = BK / 4;                  // 4-k chunks per row of a stage
    constexpr int LD = BK + 16 / (int)sizeof(T);  // LDS row stride: 16 bytes of padding
    static_assert(BK % 8 == 0, "BK must be a multiple of 8");
    constexpr int WAVES_N = 4 / WAVES_M;
    constexpr int WTM = BM / WAVES_M, WTN = BN / WAVES_N;
    constexpr int TM = WTM / 32, TN = WTN / 32;
    static_assert(TM >= 1 && TN >= 1, "wave tile must hold at least one 32x32 MFMA tile");
    static_assert(!GLU || TM == 2 || TM == 3, "GLU waves hold 32 or 48 channels (value + gate tiles)");
    constexpr int GCH = WTM / 2;  // GLU channels per wave
    __shared__ __align__(16) T As[2][BM][LD];
    __shared__ __align__(16) T Bs[2][BN][LD];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave % WAVES_M, wn = wave / WAVES_M;
    const int z = blockIdx.z;
    const int n0 = blockIdx.x * BN;
    const int m_block = blockIdx.y * (GLU ? BM / 2 : BM);
    ep.init(z);

    // Logical tile row -> physical A row (-1 when out of range).
    auto phys_row = [&](int lr) -> int {
        if constexpr (GLU) {
            const int w = lr / WTM, i = lr % WTM;
            const bool gate = i >= GCH;
            const int c = m_block + w * GCH + (gate ? i - GCH : i);
            if (c >= M) return -1;
            return gate ? M + c : c;
        } else {
            int r = m_block + lr;
            return r < M ? r : -1;
        }
    };

    // ---- operand staging: items are (row, k-quad) pairs, one float4 each ----
    // k-major: item e = (row e / KQ, quad e % KQ); m/n-major: (row e % R, quad e / R).
    constexpr int A_ITEMS = (BM * KQ + GEMM_THREADS - 1) / GEMM_THREADS;
    constexpr int B_ITEMS = (BN * KQ + GEMM_THREADS - 1) / GEMM_THREADS;
    auto a_row = [&](int e) { return AL::kmajor ? e / KQ : e % BM; };
    auto a_quad = [&](int e) { return AL::kmajor ? e % KQ : e / BM; };
    auto b_row = [&](int e) { return BL::kmajor ? e / KQ : e % BN; };
    auto b_quad = [&](int e) { return BL::kmajor ? e % KQ : e / BN; };

    // Rows of A beyond M and columns of B beyond N only feed outputs the
    // epilogue discards, so they read row / column 0 instead of being masked;
    // only k >= K must read as zero, which matters in the last k-tile alone.
    typename AL::State ast[A_ITEMS];
    typename BL::State bst[B_ITEMS];
#pragma unroll
    for (int it = 0; it < A_ITEMS; ++it) {
        int e = tid + it * GEMM_THREADS;
        int pr = e < BM * KQ ? phys_row(a_row(e)) : -1;
        ast[it] = al.setup(z, pr >= 0 ? pr : 0);
    }
#pragma unroll
    for (int it = 0; it < B_ITEMS; ++it) {
        int e = tid + it * GEMM_THREADS;
        int n = n0 + b_row(e);
        bst[it] = bl.setup(z, (e < BN * KQ && n < N) ? n : 0);
    }

    float4 areg[A_ITEMS], breg[B_ITEMS];
    // FULL: the whole k-tile lies below K and the sources allow unchecked
    // vector loads, so no per-element test is compiled into the loads.
    auto fetch = [&](const auto &ld, const auto &st, int k, auto full_tag) -> float4 {
        using L = std::decay_t<decltype(ld)>;
        constexpr bool FULL = decltype(full_tag)::value;
        if constexpr (L::kmajor) {
            if constexpr (FULL)
                return ld.load4_full(st, k);
            else
                return ld.load4(st, k, K);
        } else {
            float4 v;
            if constexpr (FULL) {
                v.x = ld.load(st, k);
                v.y = ld.load(st, k + 1);
                v.z = ld.load(st, k + 2);
                v.w = ld.load(st, k + 3);
            } else {
                v.x = k < K ? ld.load(st, k) : 0.f;
                v.y = k + 1 < K ? ld.load(st, k + 1) : 0.f;
                v.z = k + 2 < K ? ld.load(st, k + 2) : 0.f;
                v.w = k + 3 < K ? ld.load(st, k + 3) : 0.f;
            }
            return v;
        }
    };
    auto load_tiles = [&](int k0, auto full_tag) {
#pragma unroll
        for (int it = 0; it < A_ITEMS; ++it)
            areg[it] = fetch(al, ast[it], k0 + 4 * a_quad(tid + it * GEMM_THREADS), full_tag);
#pragma unroll
        for (int it = 0; it < B_ITEMS; ++it)
            breg[it] = fetch(bl, bst[it], k0 + 4 * b_quad(tid + it * GEMM_THREADS), full_tag);
    };
    const bool fast = al.fast() && bl.fast();
    auto load_next = [&](int k0) {
        if (fast && k0 + BK <= K)
            load_tiles(k0, std::true_type{});
        else
            load_tiles(k0, std::false_type{});
    };
    auto put = [&](T *dst, const float4 &v) {
        if constexpr (BF16)
            *reinterpret_cast<uint2 *>(dst) = pack_bf16x4(v);
        else
            *reinterpret_cast<float4 *>(dst) = v;
    };
    auto store_tiles = [&](int buf) {
#pragma unroll
        for (int it = 0; it < A_ITEMS; ++it) {
            int e = tid + it * GEMM_THREADS;
            if (e < BM * KQ) put(&As[buf][a_row(e)][4 * a_quad(e)], areg[it]);
        }
#pragma unroll
        for (int it = 0; it < B_ITEMS; ++it) {
            int e = tid + it * GEMM_THREADS;
            if (e < BN * KQ) put(&Bs[buf][b_row(e)][4 * b_quad(e)], breg[it]);
        }
    };

    floatx16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    const int nk = (K + BK - 1) / BK;
    load_next(0);
    store_tiles(0);
    __syncthreads();
    const int row_in = lane & 31, khalf = lane >> 5;
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < nk) load_next((kt + 1) * BK);
#ifdef DMX_GEMM_SETPRIO  // tuning builds only
        __builtin_amdgcn_s_setprio(1);
#endif
        if constexpr (BF16) {
            // Lane half h holds k = 16g + 8h .. +7 of its row for A and B alike.
#pragma unroll
            for (int g = 0; g < BK / 16; ++g) {
                bf16x8 a[TM], b[TN];
#pragma unroll
                for (int i = 0; i < TM; ++i)
                    a[i] = *reinterpret_cast<const bf16x8 *>(&As[cur][wm * WTM + i * 32 + row_in][16 * g + 8 * khalf]);
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    b[j] = *reinterpret_cast<const bf16x8 *>(&Bs[cur][wn * WTN + j * 32 + row_in][16 * g + 8 * khalf]);
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
            }
        } else {
#pragma unroll
            for (int g = 0; g < BK / 8; ++g) {
                floatx4 a[TM], b[TN];
#pragma unroll
                for (int i = 0; i < TM; ++i)
                    a[i] = *reinterpret_cast<const floatx4 *>(&As[cur][wm * WTM + i * 32 + row_in][8 * g + 4 * khalf]);
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    b[j] = *reinterpret_cast<const floatx4 *>(&Bs[cur][wn * WTN + j * 32 + row_in][8 * g + 4 * khalf]);
#pragma unroll
                for (int t = 0; t < 4; ++t)
#pragma unroll
                    for (int i = 0; i < TM; ++i)
#pragma unroll
                        for (int j = 0; j < TN; ++j)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i][t], b[j][t], acc[i][j], 0, 0, 0);
            }
        }
#ifdef DMX_GEMM_SETPRIO
        __builtin_amdgcn_s_setprio(0);
#endif
        // Interleave the MFMAs with the LDS reads and the next tile's global
        // loads (measured 2-20 % faster across the model's shapes).
        __builtin_amdgcn_iglp_opt(DMX_GEMM_IGLP);
        if (kt + 1 < nk) store_tiles(cur ^ 1);
        __syncthreads();
    }

    // ---- epilogue ----
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int n = n0 + wn * WTN + j * 32 + row_in;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int rr = 8 * (r / 4) + 4 * khalf + (r % 4);
            if constexpr (GLU) {
                // 8-row block b = 32 i + 8 (r / 4) of the wave tile; its gate
                // block b + GCH is tile gi, register gr of this same lane.
#pragma unroll
                for (int i = 0; i < TM; ++i) {
                    const int b = 32 * i + 8 * (r / 4);
                    if (b >= GCH) continue;
                    const int gi = (b + GCH) / 32, gr = (((b + GCH) % 32) / 8) * 4 + r % 4;
                    const int c = m_block + wm * GCH + 32 * i + rr;
                    if (c < M && n < N) ep.glu(z, c, n, acc[i][j][r], acc[gi][j][gr]);
                }
            } else {
#pragma unroll
                for (int i = 0; i < TM; ++i) {
                    const int m = m_block + wm * WTM + i * 32 + rr;
                    if (m < M && n < N) ep.store(z, m, n, acc[i][j][r]);
                }
            }
        }
    }
    ep.finalize(z);
}

// Launches gemm_kernel on `stream` for `batches` independent problems.
template <int BM, int BN, int WAVES_M, bool GLU, bool BF16 = false, class AL, class BL, class EP>
void launch_gemm(hipStream_t stream, int M, int N, int K, int batches, const AL &al, const BL &bl, const EP &ep) {
    if (M <= 0 || N <= 0 || batches <= 0) return;
    const int m_per_block = GLU ? BM / 2 : BM;
    dim3 grid((unsigned)ceil_div(N, BN), (unsigned)ceil_div(M, m_per_block), (unsigned)batches);
    DMX_REQUIRE(grid.y <= 65535 && grid.z <= 65535, "GEMM grid too large");
    hipLaunchKernelGGL((gemm_kernel<BM, BN, WAVES_M, GLU, BF16, AL, BL, EP>), grid, dim3(GEMM_THREADS), 0, stream, M,
                       N, K, al, bl, ep);
    DMX_LAUNCH_CHECK();
}

// ---------------------------------------------------------------------------
// Common loaders and epilogue pieces.
// ---------------------------------------------------------------------------

// Row-major matrix whose k axis is contiguous: X[z*batch_stride + row*ld + k].
struct KMajor {
    static constexpr bool kmajor = true;
    const float *p;
    int64_t ld, batch_stride;
    bool vec;  // ld and base are multiples of 4 floats: float4 loads allowed
    struct State {
        const float *row;
    };
    __device__ State setup(int z, int row) const { return {p + z * batch_stride + (int64_t)row * ld}; }
    __device__ bool fast() const { return vec; }
    __device__ float4 load4_full(const State &s, int k) const { return *reinterpret_cast<const float4 *>(s.row + k); }
    __device__ float4 load4(const State &s, int k, int K) const {
        if (vec && k + 3 < K) return *reinterpret_cast<const float4 *>(s.row + k);
        float4 v;
        v.x = k < K ? s.row[k] : 0.f;
        v.y = k + 1 < K ? s.row[k + 1] : 0.f;
        v.z = k + 2 < K ? s.row[k + 2] : 0.f;
        v.w = k + 3 < K ? s.row[k + 3] : 0.f;
        return v;
    }
};

// Row-major matrix whose m/n axis is contiguous: X[z*batch_stride + k*ld + mn].
struct MNMajor {
    static constexpr bool kmajor = false;
    const float *p;
    int64_t ld, batch_stride;
    struct State {
        const float *col;
    };
    __device__ State setup(int z, int mn) const { return {p + z * batch_stride + mn}; }
    __device__ bool fast() const { return true; }
    __device__ float load(const State &s, int k) const { return s.col[(int64_t)k * ld]; }
};

// Epilogue base: no per-problem setup, nothing to flush.
struct EpBase {
    __device__ void init(int) {}
    __device__ void finalize(int) {}
};

// Epilogue-side f64 moment accumulation: every stored value adds to (s, q),
// and finalize() reduces over the block and adds into stats[z].
struct MomentAcc {
    double s = 0.0, q = 0.0;
    __device__ void add(float v) {
        double d = v;
        s += d;
        q += d * d;
    }
    __device__ void flush(double *dst) { block_moments_atomic(s, q, dst); }
};

}  // namespace dmx
