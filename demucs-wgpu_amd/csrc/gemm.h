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
// Operand tiles go global -> registers -> LDS (double buffered, one barrier
// per BK step), so the next tile's global loads overlap this tile's MFMAs.
//
// GLU mode: each wave's two 32-row m-tiles hold the value channels c and the
// gate channels C + c of the same outputs, so GLU happens in registers and the
// 2C-channel product is never written.
#pragma once

#include "common.h"

namespace dmx {

typedef float floatx16 __attribute__((ext_vector_type(16)));

// k-tile depth. 16 measured faster than 32 at every model shape on MI355X:
// the double-buffered 128x128x16 stage (33 KB of LDS) keeps three workgroups
// per CU resident, and occupancy hides the global-load latency better than a
// deeper stage does.
#ifndef DMX_GEMM_BK
#define DMX_GEMM_BK 16
#endif
constexpr int GEMM_BK = DMX_GEMM_BK;
constexpr int GEMM_THREADS = 256;

template <int BM, int BN, int WAVES_M, bool GLU, class AL, class BL, class EP>
__global__ __launch_bounds__(GEMM_THREADS) void gemm_kernel(int M, int N, int K, AL al, BL bl, EP ep) {
    constexpr int BK = GEMM_BK;
    constexpr int KQ = BK / 4;  // float4 chunks per k-major row of a stage
    static_assert(BK % 4 == 0, "BK must be a multiple of 4");
    constexpr int WAVES_N = 4 / WAVES_M;
    constexpr int WTM = BM / WAVES_M, WTN = BN / WAVES_N;
    constexpr int TM = WTM / 32, TN = WTN / 32;
    static_assert(TM >= 1 && TN >= 1, "wave tile must hold at least one 32x32 MFMA tile");
    static_assert(!GLU || TM == 2, "GLU needs exactly one value and one gate tile per wave");
    constexpr int LDA = BM + 2, LDB = BN + 2;  // row stride = 2 mod 32 banks
    __shared__ float As[2][BK][LDA];
    __shared__ float Bs[2][BK][LDB];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave % WAVES_M, wn = wave / WAVES_M;
    const int z = blockIdx.z;
    const int n0 = blockIdx.x * BN;
    const int m_block = blockIdx.y * (GLU ? BM / 2 : BM);
    ep.init(z);

    // Logical tile row -> physical A row (-1 when out of range).
    auto phys_row = [&](int lr) -> int {
        if constexpr (GLU) {
            int w = lr / WTM, t = (lr % WTM) / 32, i = lr % 32;
            int c = m_block + w * 32 + i;
            if (c >= M) return -1;
            return t ? M + c : c;
        } else {
            int r = m_block + lr;
            return r < M ? r : -1;
        }
    };

    // ---- A operand staging ----
    // k-major sources: 4 consecutive k per thread (a float4 when aligned).
    // m-major sources: one element per thread per pass, consecutive threads on
    // consecutive rows.
    constexpr int A_KM_ITEMS = (BM * BK / 4 + GEMM_THREADS - 1) / GEMM_THREADS;
    constexpr int A_MM_ITEMS = (BM * BK + GEMM_THREADS - 1) / GEMM_THREADS;
    constexpr int B_KM_ITEMS = (BN * BK / 4 + GEMM_THREADS - 1) / GEMM_THREADS;
    constexpr int B_MM_ITEMS = (BN * BK + GEMM_THREADS - 1) / GEMM_THREADS;
    constexpr int A_REGS = AL::kmajor ? A_KM_ITEMS * 4 : A_MM_ITEMS;
    constexpr int B_REGS = BL::kmajor ? B_KM_ITEMS * 4 : B_MM_ITEMS;
    constexpr int A_STATES = AL::kmajor ? A_KM_ITEMS : A_MM_ITEMS;
    constexpr int B_STATES = BL::kmajor ? B_KM_ITEMS : B_MM_ITEMS;

    typename AL::State ast[A_STATES];
    typename BL::State bst[B_STATES];
    bool aok[A_STATES], bok[B_STATES];
#pragma unroll
    for (int it = 0; it < A_STATES; ++it) {
        int e = tid + it * GEMM_THREADS;
        int lr = AL::kmajor ? e / KQ : e % BM;
        bool in_tile = AL::kmajor ? (e < BM * BK / 4) : (e < BM * BK);
        int pr = in_tile ? phys_row(lr) : -1;
        aok[it] = pr >= 0;
        ast[it] = al.setup(z, aok[it] ? pr : 0);
    }
#pragma unroll
    for (int it = 0; it < B_STATES; ++it) {
        int e = tid + it * GEMM_THREADS;
        int lc = BL::kmajor ? e / KQ : e % BN;
        bool in_tile = BL::kmajor ? (e < BN * BK / 4) : (e < BN * BK);
        int n = n0 + lc;
        bok[it] = in_tile && n < N;
        bst[it] = bl.setup(z, bok[it] ? n : 0);
    }

    float areg[A_REGS], breg[B_REGS];

    auto load_tiles = [&](int k0) {
#pragma unroll
        for (int it = 0; it < A_STATES; ++it) {
            int e = tid + it * GEMM_THREADS;
            if constexpr (AL::kmajor) {
                int k = k0 + 4 * (e % KQ);
                float4 v = aok[it] ? al.load4(ast[it], k, K) : make_float4(0.f, 0.f, 0.f, 0.f);
                areg[4 * it + 0] = v.x;
                areg[4 * it + 1] = v.y;
                areg[4 * it + 2] = v.z;
                areg[4 * it + 3] = v.w;
            } else {
                int k = k0 + e / BM;
                areg[it] = (aok[it] && k < K) ? al.load(ast[it], k) : 0.0f;
            }
        }
#pragma unroll
        for (int it = 0; it < B_STATES; ++it) {
            int e = tid + it * GEMM_THREADS;
            if constexpr (BL::kmajor) {
                int k = k0 + 4 * (e % KQ);
                float4 v = bok[it] ? bl.load4(bst[it], k, K) : make_float4(0.f, 0.f, 0.f, 0.f);
                breg[4 * it + 0] = v.x;
                breg[4 * it + 1] = v.y;
                breg[4 * it + 2] = v.z;
                breg[4 * it + 3] = v.w;
            } else {
                int k = k0 + e / BN;
                breg[it] = (bok[it] && k < K) ? bl.load(bst[it], k) : 0.0f;
            }
        }
    };

    auto store_tiles = [&](int buf) {
#pragma unroll
        for (int it = 0; it < A_STATES; ++it) {
            int e = tid + it * GEMM_THREADS;
            if constexpr (AL::kmajor) {
                if (e < BM * BK / 4) {
                    int lr = e / KQ, kk = 4 * (e % KQ);
#pragma unroll
                    for (int j = 0; j < 4; ++j) As[buf][kk + j][lr] = areg[4 * it + j];
                }
            } else {
                if (e < BM * BK) As[buf][e / BM][e % BM] = areg[it];
            }
        }
#pragma unroll
        for (int it = 0; it < B_STATES; ++it) {
            int e = tid + it * GEMM_THREADS;
            if constexpr (BL::kmajor) {
                if (e < BN * BK / 4) {
                    int lc = e / KQ, kk = 4 * (e % KQ);
#pragma unroll
                    for (int j = 0; j < 4; ++j) Bs[buf][kk + j][lc] = breg[4 * it + j];
                }
            } else {
                if (e < BN * BK) Bs[buf][e / BN][e % BN] = breg[it];
            }
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
    load_tiles(0);
    store_tiles(0);
    __syncthreads();
    const int row_in = lane & 31, khalf = lane >> 5;
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < nk) load_tiles((kt + 1) * BK);
#pragma unroll
        for (int s = 0; s < BK / 2; ++s) {
            float a[TM], b[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i) a[i] = As[cur][2 * s + khalf][wm * WTM + i * 32 + row_in];
#pragma unroll
            for (int j = 0; j < TN; ++j) b[j] = Bs[cur][2 * s + khalf][wn * WTN + j * 32 + row_in];
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], b[j], acc[i][j], 0, 0, 0);
        }
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
                const int c = m_block + wm * 32 + rr;
                if (c < M && n < N) ep.glu(z, c, n, acc[0][j][r], acc[1][j][r]);
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
template <int BM, int BN, int WAVES_M, bool GLU, class AL, class BL, class EP>
void launch_gemm(hipStream_t stream, int M, int N, int K, int batches, const AL &al, const BL &bl, const EP &ep) {
    if (M <= 0 || N <= 0 || batches <= 0) return;
    const int m_per_block = GLU ? BM / 2 : BM;
    dim3 grid((unsigned)ceil_div(N, BN), (unsigned)ceil_div(M, m_per_block), (unsigned)batches);
    DMX_REQUIRE(grid.y <= 65535 && grid.z <= 65535, "GEMM grid too large");
    hipLaunchKernelGGL((gemm_kernel<BM, BN, WAVES_M, GLU, AL, BL, EP>), grid, dim3(GEMM_THREADS), 0, stream, M, N,
                       K, al, bl, ep);
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
