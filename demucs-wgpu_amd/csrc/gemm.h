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

// MFMA input precision of gemm_kernel (its PREC parameter): fp32 (0), bf16
// (1), or three bf16 planes per operand (3: x = x0 + x1 + x2, the six plane
// products with i + j < 3 summed in fp32, an fp32-accurate product; the
// loader splits each value into its planes as it stores it in LDS).
// Stage element type, depth and planes: fp32 stages BK = 16 floats per row;
// bf16 stages 32 (one v_mfma_f32_32x32x16_bf16 per 16, operands 8 bf16 per
// lane); three planes stage 16 per plane.
template <int PREC>
struct GemmStage {
    using T = float;
    static constexpr int BK = GEMM_BK;
    static constexpr int PLANES = 1;
};
template <>
struct GemmStage<1> {
    using T = unsigned short;
    static constexpr int BK = 32;
    static constexpr int PLANES = 1;
};
template <>
struct GemmStage<3> {
    using T = unsigned short;
    static constexpr int BK = 16;
    static constexpr int PLANES = 3;
};

// Four values -> three bf16 planes (round to nearest even at each step), as
// bits, four per uint2: two pairs, one v_cvt_pk_bf16_f32 per pair and plane.
__device__ __forceinline__ void split_planes4(float4 v, uint2 (&out)[3]) {
    unsigned lo[3], hi[3];
    split_pair_planes<3>(v.x, v.y, lo);
    split_pair_planes<3>(v.z, v.w, hi);
#pragma unroll
    for (int q = 0; q < 3; ++q) out[q] = make_uint2(lo[q], hi[q]);
}

// An m/n-major loader may fetch four consecutive k of one column at once
// (load_quad, k a multiple of 4); when K is a multiple of 4 a quad is either
// wholly below K or wholly past it.
template <class L, class = void>
struct has_load_quad : std::false_type {};
template <class L>
struct has_load_quad<L, std::void_t<decltype(&L::load_quad)>> : std::true_type {};

// An m/n-major loader may also split a quad in two: load_raw(state, k)
// only issues the loads (returning the loaded values as its Raw type) and
// finish(state, raw, k) turns them into the operand (a skip add, a norm).
// The kernel issues load_raw before a k-tile's MFMAs and calls finish after
// them, just before the LDS store, so the loads are in flight during the
// MFMAs instead of being waited for on the spot. zero_raw() finishes to 0.
template <class L, class = void>
struct has_load_raw : std::false_type {};
template <class L>
struct has_load_raw<L, std::void_t<typename L::Raw>> : std::true_type {};
// An epilogue may take a wave's whole fragments of a tile that lies wholly in
// range (store_frags, announced by a `frags` member): it can then hoist the
// per-column and per-row index arithmetic out of the element loop.
template <class E, class = void>
struct has_store_frags : std::false_type {};
template <class E>
struct has_store_frags<E, std::void_t<decltype(E::frags)>> : std::true_type {};

template <class L, bool = has_load_raw<L>::value>
struct raw_of {
    using type = float4;
};
template <class L>
struct raw_of<L, true> {
    using type = typename L::Raw;
};

// Row addressing of a k-major fp32 matrix for the direct-to-LDS kernel:
// row r of problem z starts at p + z * batch_stride + r * ld.
struct KMajorRows {
    const float *p;
    int64_t ld, batch_stride;
    __device__ const float *row(int z, int r) const { return p + z * batch_stride + (int64_t)r * ld; }
};

// This block's (column tile, row tile, batch) in the XCD-contiguous order of
// the x-fastest grid: an XCD runs consecutive column tiles of one row panel.
__device__ __forceinline__ void block_tile(int &bx, int &by, int &z) {
    const int nx = gridDim.x, ny = gridDim.y;
    const int lb = xcd_contiguous(blockIdx.x + nx * (blockIdx.y + ny * blockIdx.z), nx * ny * gridDim.z);
    bx = lb % nx;
    by = (lb / nx) % ny;
    z = lb / (nx * ny);
}

template <int BM, int BN, int WAVES_M, bool GLU, int PREC, class AL, class BL, class EP>
__global__ __launch_bounds__(GEMM_THREADS) void gemm_kernel(int M, int N, int K, AL al, BL bl, EP ep) {
    using T = typename GemmStage<PREC>::T;
    constexpr int BK = GemmStage<PREC>::BK;
    constexpr int NP = GemmStage<PREC>::PLANES;
    constexpr int KQ = BK / 4;                  // 4-k chunks per row of a stage
    constexpr int LD = BK + 16 / (int)sizeof(T);  // LDS row stride: 16 bytes of padding
    static_assert(BK % 8 == 0, "BK must be a multiple of 8");
    constexpr int WAVES_N = 4 / WAVES_M;
    constexpr int WTM = BM / WAVES_M, WTN = BN / WAVES_N;
    constexpr int TM = WTM / 32, TN = WTN / 32;
    static_assert(TM >= 1 && TN >= 1, "wave tile must hold at least one 32x32 MFMA tile");
    static_assert(!GLU || TM == 2 || TM == 3, "GLU waves hold 32 or 48 channels (value + gate tiles)");
    constexpr int GCH = WTM / 2;  // GLU channels per wave
    __shared__ __align__(16) T As[2][NP][BM][LD];
    __shared__ __align__(16) T Bs[2][NP][BN][LD];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave % WAVES_M, wn = wave / WAVES_M;
    int bx, by, z;
    block_tile(bx, by, z);
    const int n0 = bx * BN;
    const int m_block = by * (GLU ? BM / 2 : BM);
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

    constexpr bool B_RAW = has_load_raw<BL>::value;
    float4 areg[A_ITEMS];
    typename raw_of<BL>::type breg[B_ITEMS];
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
        } else if constexpr (has_load_quad<L>::value) {
            if (FULL || k < K) return ld.load_quad(st, k);
            return make_float4(0.f, 0.f, 0.f, 0.f);
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
        for (int it = 0; it < B_ITEMS; ++it) {
            const int k = k0 + 4 * b_quad(tid + it * GEMM_THREADS);
            if constexpr (B_RAW)
                breg[it] = (decltype(full_tag)::value || k < K) ? bl.load_raw(bst[it], k) : bl.zero_raw();
            else
                breg[it] = fetch(bl, bst[it], k, full_tag);
        }
    };
    const bool fast = al.fast() && bl.fast();
    auto load_next = [&](int k0) {
        if (fast && k0 + BK <= K)
            load_tiles(k0, std::true_type{});
        else
            load_tiles(k0, std::false_type{});
    };
    // Four values of row r, k-quad q into LDS (plane stride PS elements).
    auto put = [&](T *dst, int64_t ps, const float4 &v) {
        if constexpr (PREC == 3) {
            uint2 pl[3];
            split_planes4(v, pl);
#pragma unroll
            for (int q = 0; q < 3; ++q) *reinterpret_cast<uint2 *>(dst + q * ps) = pl[q];
        } else if constexpr (PREC == 1) {
            (void)ps;
            *reinterpret_cast<uint2 *>(dst) = pack_bf16x4(v);
        } else {
            (void)ps;
            *reinterpret_cast<float4 *>(dst) = v;
        }
    };
    auto store_tiles = [&](int buf, int k0) {
#pragma unroll
        for (int it = 0; it < A_ITEMS; ++it) {
            int e = tid + it * GEMM_THREADS;
            if (e < BM * KQ) put(&As[buf][0][a_row(e)][4 * a_quad(e)], BM * LD, areg[it]);
        }
#pragma unroll
        for (int it = 0; it < B_ITEMS; ++it) {
            int e = tid + it * GEMM_THREADS;
            if (e < BN * KQ) {
                if constexpr (B_RAW)
                    put(&Bs[buf][0][b_row(e)][4 * b_quad(e)], BN * LD, bl.finish(bst[it], breg[it], k0 + 4 * b_quad(e)));
                else
                    put(&Bs[buf][0][b_row(e)][4 * b_quad(e)], BN * LD, breg[it]);
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
    load_next(0);
    store_tiles(0, 0);
    __syncthreads();
    const int row_in = lane & 31, khalf = lane >> 5;
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < nk) load_next((kt + 1) * BK);
#ifdef DMX_GEMM_SETPRIO  // tuning builds only
        __builtin_amdgcn_s_setprio(1);
#endif
        if constexpr (PREC == 3) {
            // Three planes: lane half h holds k = 16g + 8h .. +7 of its row in
            // every plane; the six plane products with i + j < 3, smallest
            // first.
#pragma unroll
            for (int g = 0; g < BK / 16; ++g) {
                bf16x8 a[3][TM], b[3][TN];
#pragma unroll
                for (int q = 0; q < 3; ++q) {
#pragma unroll
                    for (int i = 0; i < TM; ++i)
                        a[q][i] = *reinterpret_cast<const bf16x8 *>(
                            &As[cur][q][wm * WTM + i * 32 + row_in][16 * g + 8 * khalf]);
#pragma unroll
                    for (int j = 0; j < TN; ++j)
                        b[q][j] = *reinterpret_cast<const bf16x8 *>(
                            &Bs[cur][q][wn * WTN + j * 32 + row_in][16 * g + 8 * khalf]);
                }
                constexpr int pa[6] = {2, 1, 0, 1, 0, 0}, pb[6] = {0, 1, 2, 0, 1, 0};
#pragma unroll
                for (int t = 0; t < 6; ++t)
#pragma unroll
                    for (int i = 0; i < TM; ++i)
#pragma unroll
                        for (int j = 0; j < TN; ++j)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[pa[t]][i], b[pb[t]][j], acc[i][j],
                                                                                0, 0, 0);
            }
        } else if constexpr (PREC == 1) {
            // Lane half h holds k = 16g + 8h .. +7 of its row for A and B alike.
#pragma unroll
            for (int g = 0; g < BK / 16; ++g) {
                bf16x8 a[TM], b[TN];
#pragma unroll
                for (int i = 0; i < TM; ++i)
                    a[i] = *reinterpret_cast<const bf16x8 *>(&As[cur][0][wm * WTM + i * 32 + row_in][16 * g + 8 * khalf]);
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    b[j] = *reinterpret_cast<const bf16x8 *>(&Bs[cur][0][wn * WTN + j * 32 + row_in][16 * g + 8 * khalf]);
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
                    a[i] = *reinterpret_cast<const floatx4 *>(&As[cur][0][wm * WTM + i * 32 + row_in][8 * g + 4 * khalf]);
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    b[j] = *reinterpret_cast<const floatx4 *>(&Bs[cur][0][wn * WTN + j * 32 + row_in][8 * g + 4 * khalf]);
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
        if (kt + 1 < nk) store_tiles(cur ^ 1, (kt + 1) * BK);
        __syncthreads();
    }

    // ---- epilogue ----
    if constexpr (has_store_frags<EP>::value) {
        if constexpr (GLU) {
            if (m_block + BM / 2 <= M && n0 + BN <= N) {
                ep.template glu_frags<GCH>(z, m_block + wm * GCH, n0 + wn * WTN, row_in, khalf, acc);
                ep.finalize(z);
                return;
            }
        } else {
            if (m_block + BM <= M && n0 + BN <= N) {
                ep.store_frags(z, m_block + wm * WTM, n0 + wn * WTN, row_in, khalf, acc);
                ep.finalize(z);
                return;
            }
        }
    }
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
template <int BM, int BN, int WAVES_M, bool GLU, int PREC = 0, class AL, class BL, class EP>
void launch_gemm(hipStream_t stream, int M, int N, int K, int batches, const AL &al, const BL &bl, const EP &ep) {
    if (M <= 0 || N <= 0 || batches <= 0) return;
    const int m_per_block = GLU ? BM / 2 : BM;
    dim3 grid((unsigned)ceil_div(N, BN), (unsigned)ceil_div(M, m_per_block), (unsigned)batches);
    DMX_REQUIRE(grid.y <= 65535 && grid.z <= 65535, "GEMM grid too large");
    hipLaunchKernelGGL((gemm_kernel<BM, BN, WAVES_M, GLU, PREC, AL, BL, EP>), grid, dim3(GEMM_THREADS), 0, stream, M,
                       N, K, al, bl, ep);
    DMX_LAUNCH_CHECK();
}

// ---------------------------------------------------------------------------
// Direct-to-LDS GEMM for two k-major fp32 operands (the transformer linears:
// activations (M, K) times weights (N, K)).
//
// The operand tiles go from global memory straight into LDS with
// global_load_lds_dwordx4: no staging registers and no ds_write, so STAGES
// k-tiles can be in flight at once while the MFMAs work on the oldest one.
// One DMA instruction fills 1 KB of LDS, lane l writing bytes [16 l, 16 l + 16):
// sixteen 64-byte rows (BK = 16 floats) of four 16-byte chunks. Lane l fetches
// row l / 4 of its group and, in slot l % 4, the chunk (l % 4) ^ swz(row), so
// a ds_read_b128 of one logical chunk over 16 consecutive rows touches 16
// distinct bank quads (and 8 consecutive rows 8 distinct ones): the XOR
// swizzle makes the MFMA operand reads conflict-free without padding, which a
// DMA row layout cannot have.
//
// Waits: each wave counts its own DMA instructions with vmcnt (loads retire in
// order); the barrier after the wait makes every wave's part of the k-tile
// visible, and it also guarantees that the buffer refilled next was read by
// every wave in the previous iteration. The operand reads are issued as
// inline ds_read_b128 with explicit lgkmcnt waits: the compiler cannot tell
// which stage a read touches, and would otherwise put a vmcnt(0) (wait for
// every DMA in flight) in front of each of them, which serialises the
// pipeline.
// ---------------------------------------------------------------------------

__device__ __forceinline__ int dma_swz(int r) { return ((r >> 1) ^ (r >> 3)) & 3; }

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// One DMA instruction: lane l copies 16 bytes from src to dst + 16 l bytes
// (dst is wave-uniform). A plain __device__ function, so the device-only
// builtin never sits in a lambda that the host side also analyses.
__device__ __forceinline__ void dma_b128(const float *src, float *dst) {
    __builtin_amdgcn_global_load_lds(src, dst, 16, 0, 0);
}

// 16 bytes from LDS (p points into a __shared__ array).
__device__ __forceinline__ floatx4 lds_read_b128(const float *p) {
    floatx4 v;
    const unsigned addr = (unsigned)(uintptr_t)p;  // low 32 bits of a shared address = LDS offset
    asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr) : "memory");
    return v;
}

// Passes values through an empty volatile asm: no use of them can be
// scheduled before the asm statements that precede this one.
template <int TA, int TB>
__device__ __forceinline__ void pin_regs(floatx4 (&a)[TA], floatx4 (&b)[TB]) {
#pragma unroll
    for (int i = 0; i < TA; ++i) asm volatile("" : "+v"(a[i]));
#pragma unroll
    for (int j = 0; j < TB; ++j) asm volatile("" : "+v"(b[j]));
}

// Waits for every LDS read in flight, then pins the values read.
template <int TA, int TB>
__device__ __forceinline__ void lds_wait(floatx4 (&a)[TA], floatx4 (&b)[TB]) {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    pin_regs(a, b);
}

// Waves per SIMD the register allocation leaves room for. Two (four k-tiles
// in flight, 64 KB of LDS per block) measured 1-3 % faster on the model's
// linears than three (three k-tiles, registers capped at 168).
#ifndef DMX_DMA_WPE
#define DMX_DMA_WPE 2
#endif
template <int BM, int BN, int WAVES_M, int STAGES, class EP>
__global__ __launch_bounds__(GEMM_THREADS) __attribute__((amdgpu_waves_per_eu(DMX_DMA_WPE))) void gemm_dma_kernel(int M, int N, int K, KMajorRows al, KMajorRows bl,
                                                                EP ep) {
    constexpr int BK = 16;                     // two MFMA k-groups of 8 per k-tile
    constexpr int ROWS = BM + BN;              // staged rows per k-tile: A rows, then B rows
    constexpr int INSTR = ROWS / 16;           // 1 KB DMA instructions per k-tile
    constexpr int PER_WAVE = INSTR / 4;
    constexpr int STAGE = ROWS * BK;           // floats per k-tile
    static_assert(BM % 16 == 0 && BN % 16 == 0 && INSTR % 4 == 0, "tile rows must fill whole DMA instructions");
    static_assert(STAGES >= 2 && PER_WAVE * (STAGES - 2) < 64, "pipeline depth");
    constexpr int WAVES_N = 4 / WAVES_M;
    constexpr int WTM = BM / WAVES_M, WTN = BN / WAVES_N;
    constexpr int TM = WTM / 32, TN = WTN / 32;
    static_assert(TM >= 1 && TN >= 1, "wave tile must hold at least one 32x32 MFMA tile");
    __shared__ __align__(16) float lds[STAGES * STAGE];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave % WAVES_M, wn = wave / WAVES_M;
    int bx, by, z;
    block_tile(bx, by, z);
    const int n0 = bx * BN, m0 = by * BM;
    ep.init(z);

    // Sources of this lane's DMA slots. Rows past M / N repeat the last row:
    // they only feed outputs the epilogue discards.
    const int grow = lane >> 2, gchunk = (lane & 3) ^ dma_swz(lane >> 2);
    const float *src[PER_WAVE];
#pragma unroll
    for (int i = 0; i < PER_WAVE; ++i) {
        const int r = 16 * (wave + 4 * i) + grow;
        if (r < BM)
            src[i] = al.row(z, min(m0 + r, M - 1)) + 4 * gchunk;
        else
            src[i] = bl.row(z, min(n0 + r - BM, N - 1)) + 4 * gchunk;
    }
    auto issue = [&](int buf, int k0) {
#pragma unroll
        for (int i = 0; i < PER_WAVE; ++i)
            dma_b128(src[i] + k0, &lds[buf * STAGE + (wave + 4 * i) * 256]);
    };

    floatx16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    // LDS float offsets of this lane's operand rows (row * BK), and their swizzle.
    const int row_in = lane & 31, khalf = lane >> 5;
    int a_off[TM], a_swz[TM], b_off[TN], b_swz[TN];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const int r = wm * WTM + i * 32 + row_in;
        a_off[i] = r * BK;
        a_swz[i] = dma_swz(r & 15);
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int r = BM + wn * WTN + j * 32 + row_in;
        b_off[j] = r * BK;
        b_swz[j] = dma_swz(r & 15);
    }

    const int nk = K / BK;
#pragma unroll
    for (int st = 0; st < STAGES - 1; ++st)
        if (st < nk) issue(st, st * BK);
    for (int kt = 0; kt < nk; ++kt) {
        if (kt + STAGES - 2 < nk)
            wait_vmcnt<PER_WAVE * (STAGES - 2)>();
        else
            wait_vmcnt<0>();
        __builtin_amdgcn_s_barrier();
        if (kt + STAGES - 1 < nk) issue((kt + STAGES - 1) % STAGES, (kt + STAGES - 1) * BK);
        const float *stage = lds + (kt % STAGES) * STAGE;
        // Group g holds k = 8g .. 8g + 7; lane half h reads its logical chunk
        // 2g + h (k = 8g + 4h .. +3). Group 1's reads fly during group 0's MFMAs.
        floatx4 a[2][TM], b[2][TN];
        auto read_group = [&](int g) {
            const int c = 2 * g + khalf;
#pragma unroll
            for (int i = 0; i < TM; ++i) a[g][i] = lds_read_b128(stage + a_off[i] + 4 * (c ^ a_swz[i]));
#pragma unroll
            for (int j = 0; j < TN; ++j) b[g][j] = lds_read_b128(stage + b_off[j] + 4 * (c ^ b_swz[j]));
        };
        auto mfma_group = [&](int g) {
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[g][i][t], b[g][j][t], acc[i][j], 0, 0, 0);
        };
        read_group(0);
        lds_wait(a[0], b[0]);
        read_group(1);
        pin_regs(a[0], b[0]);  // keeps group 0's MFMAs behind group 1's reads
#ifdef DMX_DMA_SETPRIO  // tuning builds only
        __builtin_amdgcn_s_setprio(1);
#endif
        mfma_group(0);
        __builtin_amdgcn_sched_barrier(0);  // ... and group 1's wait behind group 0's MFMAs
        lds_wait(a[1], b[1]);
        mfma_group(1);
#ifdef DMX_DMA_SETPRIO
        __builtin_amdgcn_s_setprio(0);
#endif
    }

    if (m0 + BM <= M && n0 + BN <= N) {
        // Whole tile in range: the epilogue takes the wave's fragments at once
        // (and can issue all of its loads before the first use).
        ep.store_frags(z, m0 + wm * WTM, n0 + wn * WTN, row_in, khalf, acc);
    } else {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int n = n0 + wn * WTN + j * 32 + row_in;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int rr = 8 * (r / 4) + 4 * khalf + (r % 4);
#pragma unroll
                for (int i = 0; i < TM; ++i) {
                    const int m = m0 + wm * WTM + i * 32 + rr;
                    if (m < M && n < N) ep.store(z, m, n, acc[i][j][r]);
                }
            }
        }
    }
    ep.finalize(z);
}

// Launches gemm_dma_kernel; K must be a multiple of 16 and both operands
// 16-byte aligned with row strides a multiple of 4 floats.
template <int BM, int BN, int WAVES_M, int STAGES, class EP>
void launch_gemm_dma(hipStream_t stream, int M, int N, int K, int batches, const KMajorRows &al, const KMajorRows &bl,
                     const EP &ep) {
    if (M <= 0 || N <= 0 || batches <= 0) return;
    DMX_REQUIRE(K % 16 == 0 && K > 0, "gemm_dma: K must be a positive multiple of 16");
    dim3 grid((unsigned)ceil_div(N, BN), (unsigned)ceil_div(M, BM), (unsigned)batches);
    DMX_REQUIRE(grid.y <= 65535 && grid.z <= 65535, "GEMM grid too large");
    hipLaunchKernelGGL((gemm_dma_kernel<BM, BN, WAVES_M, STAGES, EP>), grid, dim3(GEMM_THREADS), 0, stream, M, N, K,
                       al, bl, ep);
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
