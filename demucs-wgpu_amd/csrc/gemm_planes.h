// gemm_planes.h — GEMMs on the bf16 matrix cores over operands stored as
// bf16 planes.
//
// An fp32 value x is held as P bf16 planes, x = x_0 + x_1 + ... + x_{P-1}:
// x_0 = bf16(x), x_1 = bf16(x - x_0), x_2 = bf16(x - x_0 - x_1), each rounded
// to nearest even. The residual after each plane is exact in fp32, and each
// plane carries the next 8 significant bits, so three planes hold all 24 bits
// of x (split_planes below). A dot product of two split operands is the sum
// of the plane products a_i b_j; with P = 3 the six products with i + j <= 2
// are kept. The dropped ones (a_1 b_2, a_2 b_1, a_2 b_2) are below 2^-25 of
// |a b| each, under the 2^-24 rounding of an fp32 product, and every product
// of two bf16 values is exact in the fp32 accumulator of
// v_mfma_f32_32x32x16_bf16. So P = 3 computes an fp32 GEMM to fp32 accuracy
// with six bf16 MFMAs per k-step of 16 where the fp32 matrix cores need eight
// v_mfma_f32_32x32x2f32 at twice the cycles each: 2.7x the throughput bound
// on MI355X (2.5 PFLOP/s dense bf16 / 6 against 157.3 TFLOP/s fp32).
// P = 1 is a plain bf16 GEMM (bf16 inputs, fp32 accumulation).
//
// The kernel is the direct-to-LDS design of gemm_dma_kernel (gemm.h) over
// rows of 16, 32 or 64 bf16 per k-tile (one, two or four MFMA k-groups):
// global_load_lds_dwordx4 fills LDS with no staging registers, STAGES k-tiles
// in flight, an XOR swizzle of a row's 16-byte chunks keeps the operand reads
// conflict-free, and one barrier per k-tile sits between the last two
// k-groups' MFMAs. A stage holds the P planes of the A rows, then the P
// planes of the B rows. Four or eight waves per workgroup.
#pragma once

#include "gemm.h"

namespace dmx {

// x -> P bf16 planes (bits), round-to-nearest-even at each step.
template <int P>
__device__ __forceinline__ void split_planes(float x, unsigned short (&out)[P]) {
#pragma unroll
    for (int q = 0; q < P; ++q) {
        const __bf16 h = (__bf16)x;
        out[q] = __builtin_bit_cast(unsigned short, h);
        x -= (float)h;
    }
}

// Row addressing of the planes of a k-major matrix: plane q of row r of
// problem z starts at p + q * plane_stride + z * batch_stride + r * ld
// (bf16 elements).
struct PlaneRows {
    const unsigned short *p;
    int64_t ld, batch_stride, plane_stride;
    __device__ const unsigned short *row(int z, int q, int r) const {
        return p + q * plane_stride + z * batch_stride + (int64_t)r * ld;
    }
};

__device__ __forceinline__ void dma_b128(const unsigned short *src, unsigned short *dst) {
    __builtin_amdgcn_global_load_lds(src, dst, 16, 0, 0);
}

__device__ __forceinline__ floatx4 lds_read_b128(const unsigned short *p) {
    floatx4 v;
    const unsigned addr = (unsigned)(uintptr_t)p;
    asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr) : "memory");
    return v;
}

// Plane products kept for P planes: (i, j) with i + j < P.
template <int P>
struct PlanePairs {
    static constexpr int count = P * (P + 1) / 2;
    static constexpr int a(int t) {
        int i = 0;
        for (int s = 0; s < P; ++s)
            for (int j = 0; j + s < P; ++j, ++i)
                if (i == t) return s;
        return 0;
    }
    static constexpr int b(int t) {
        int i = 0;
        for (int s = 0; s < P; ++s)
            for (int j = 0; j + s < P; ++j, ++i)
                if (i == t) return j;
        return 0;
    }
};

extern __shared__ __align__(16) unsigned short gemm_planes_lds[];

// Swizzle of the 16-byte chunks of a staged row; r is the row's index in
// its DMA instruction's group of 1024 / (2 BK) rows. The reads of one
// logical chunk over 8 consecutive rows must land on distinct 16-byte slots
// of a 128-byte bank window, and over 16 consecutive rows on distinct slots
// of a 256-byte one:
// - 32-byte rows (BK = 16, two chunks): c ^ (bit 2 ^ bit 3 of r);
// - 64-byte rows (BK = 32, four chunks): gemm_dma_kernel's dma_swz;
// - 128-byte rows (BK = 64, eight chunks): c ^ ((r ^ (r >> 3)) & 7).
template <int BK>
__device__ __forceinline__ int planes_swz(int r) {
    if constexpr (BK == 64)
        return (r ^ (r >> 3)) & 7;
    else if constexpr (BK == 32)
        return dma_swz(r & 15);
    else
        return ((r >> 2) ^ (r >> 3)) & 1;
}

// Waves per SIMD the register allocation leaves room for.
#ifndef DMX_PLANES_WPE
#define DMX_PLANES_WPE 2
#endif

template <int BM, int BN, int WAVES_M, int STAGES, int P, int BK, int NW, class EP>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(DMX_PLANES_WPE))) void gemm_planes_kernel(
    int M, int N, int K, PlaneRows al, PlaneRows bl, EP ep) {
    static_assert(BK == 16 || BK == 32 || BK == 64, "k-tile of one, two or four MFMA k-groups");
    static_assert(BK == 16 || (BK / 16) % 2 == 0, "an even number of k-groups per k-tile");
    constexpr int G = BK / 16;              // MFMA k-groups per k-tile
    constexpr int CH = BK / 8;              // 16-byte chunks per staged row
    constexpr int RPI = 64 / CH;            // rows per 1 KB DMA instruction
    constexpr int AROWS = P * BM;           // staged rows: A planes, then B planes
    constexpr int ROWS = P * (BM + BN);
    constexpr int INSTR = ROWS / RPI;       // DMA instructions per k-tile
    constexpr int PER_WAVE = INSTR / NW;
    constexpr int STAGE = ROWS * BK;        // bf16 per k-tile
    static_assert(ROWS % (NW * RPI) == 0, "tile rows must fill whole DMA instructions on every wave");
    static_assert(NW == 4 || NW == 8, "four or eight waves");
    constexpr int WAVES_N = NW / WAVES_M;
    constexpr int WTM = BM / WAVES_M, WTN = BN / WAVES_N;
    constexpr int TM = WTM / 32, TN = WTN / 32;
    static_assert(TM >= 1 && TN >= 1, "wave tile must hold at least one 32x32 MFMA tile");
    // BK = 16 reads the next k-tile's operands during this one's MFMAs, so
    // the tile after that must already be in flight: three stages at least.
    static_assert(G > 1 ? (STAGES >= 2 && PER_WAVE * (STAGES - 2) < 64)
                           : (STAGES >= 3 && PER_WAVE * (STAGES - 2) < 64),
                  "pipeline depth");
    using PP = PlanePairs<P>;
    unsigned short *lds = gemm_planes_lds;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave % WAVES_M, wn = wave / WAVES_M;
    int bx, by, z;
    block_tile(bx, by, z);
    const int n0 = bx * BN, m0 = by * BM;
    ep.init(z);

    // Sources of this lane's DMA slots; rows past M / N repeat the last row
    // (they only feed outputs the epilogue discards).
    const int grow = lane / CH, gchunk = (lane % CH) ^ planes_swz<BK>(lane / CH);
    const unsigned short *src[PER_WAVE];
#pragma unroll
    for (int i = 0; i < PER_WAVE; ++i) {
        const int r = RPI * (wave + NW * i) + grow;
        if (r < AROWS)
            src[i] = al.row(z, r / BM, min(m0 + r % BM, M - 1)) + 8 * gchunk;
        else
            src[i] = bl.row(z, (r - AROWS) / BN, min(n0 + (r - AROWS) % BN, N - 1)) + 8 * gchunk;
    }
    auto issue = [&](int buf, int k0) {
#pragma unroll
        for (int i = 0; i < PER_WAVE; ++i) dma_b128(src[i] + k0, lds + buf * STAGE + (wave + NW * i) * 512);
    };

    floatx16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    // LDS offsets (bf16) of this lane's plane-0 operand rows and their
    // swizzle; plane q of A sits q * BM rows further, plane q of B q * BN.
    const int row_in = lane & 31, khalf = lane >> 5;
    int a_off[TM], a_swz[TM], b_off[TN], b_swz[TN];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const int r = wm * WTM + i * 32 + row_in;
        a_off[i] = r * BK;
        a_swz[i] = planes_swz<BK>(r % RPI);
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int r = AROWS + wn * WTN + j * 32 + row_in;
        b_off[j] = r * BK;
        b_swz[j] = planes_swz<BK>(r % RPI);
    }
    // Plane offsets are whole multiples of 32 rows, so a row's swizzle is the
    // same in every plane.

    // Operand fragments of one MFMA k-group: lane half h reads its logical
    // chunk 2g + h (k = 16 g + 8 h .. + 7) of every plane.
    auto read_group = [&](const unsigned short *stage, int g, floatx4 (&a)[P * TM], floatx4 (&b)[P * TN]) {
        const int c = 2 * g + khalf;
#pragma unroll
        for (int q = 0; q < P; ++q) {
#pragma unroll
            for (int i = 0; i < TM; ++i)
                a[q * TM + i] = lds_read_b128(stage + a_off[i] + q * BM * BK + 8 * (c ^ a_swz[i]));
#pragma unroll
            for (int j = 0; j < TN; ++j)
                b[q * TN + j] = lds_read_b128(stage + b_off[j] + q * BN * BK + 8 * (c ^ b_swz[j]));
        }
    };
    auto mfma_group = [&](const floatx4 (&a)[P * TM], const floatx4 (&b)[P * TN]) {
#pragma unroll
        for (int t = 0; t < PP::count; ++t)
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                        __builtin_bit_cast(bf16x8, a[PP::a(t) * TM + i]),
                        __builtin_bit_cast(bf16x8, b[PP::b(t) * TN + j]), acc[i][j], 0, 0, 0);
    };

    const int nk = K / BK;
#pragma unroll
    for (int st = 0; st < STAGES - 1; ++st)
        if (st < nk) issue(st, st * BK);

    if constexpr (G > 1) {
        // All STAGES buffers start filling at once. Iteration kt issues its
        // groups' MFMAs with group g + 1's reads in flight during group g's.
        // Once the second-to-last group's MFMAs are issued, the wave waits
        // for the last group's reads and for tile kt + 1's DMA, meets the
        // other waves at the barrier (after which every wave is done with
        // tile kt's buffer, which then takes tile kt + STAGES), and starts
        // reading tile kt + 1's first group: the barrier and those reads
        // overlap the MFMAs in the pipe and the last group's.
        static_assert(PER_WAVE * (STAGES - 1) < 64, "pipeline depth");
        if (STAGES - 1 < nk) issue(STAGES - 1, (STAGES - 1) * BK);
        if (nk >= STAGES)
            wait_vmcnt<PER_WAVE * (STAGES - 1)>();
        else
            wait_vmcnt<0>();
        __builtin_amdgcn_s_barrier();
        floatx4 fa[2][P * TM], fb[2][P * TN];
        read_group(lds, 0, fa[0], fb[0]);
        lds_wait(fa[0], fb[0]);
        read_group(lds, 1, fa[1], fb[1]);
        for (int kt = 0; kt < nk; ++kt) {
            const unsigned short *stage = lds + (kt % STAGES) * STAGE;
            const unsigned short *next = lds + ((kt + 1) % STAGES) * STAGE;
#pragma unroll
            for (int g = 0; g < G; ++g) {
                pin_regs(fa[g & 1], fb[g & 1]);
                mfma_group(fa[g & 1], fb[g & 1]);
                __builtin_amdgcn_sched_barrier(0);
                if (g < G - 2) {
                    lds_wait(fa[(g + 1) & 1], fb[(g + 1) & 1]);
                    read_group(stage, g + 2, fa[g & 1], fb[g & 1]);
                } else if (g == G - 2) {
                    lds_wait(fa[(g + 1) & 1], fb[(g + 1) & 1]);
                    if (kt + 1 < nk) {
                        if (kt + STAGES - 1 < nk)
                            wait_vmcnt<PER_WAVE * (STAGES - 2)>();
                        else
                            wait_vmcnt<0>();
                        __builtin_amdgcn_s_barrier();
                        if (kt + STAGES < nk) issue(kt % STAGES, (kt + STAGES) * BK);
                        read_group(next, 0, fa[g & 1], fb[g & 1]);
                    }
                } else if (kt + 1 < nk) {
                    // Group 0 of tile kt + 1 went into the registers of group
                    // G - 2 (G is even); group 1 takes this group's.
                    lds_wait(fa[0], fb[0]);
                    read_group(next, 1, fa[1], fb[1]);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    } else {
        // One k-group per k-tile; the next tile's reads fly during this
        // tile's MFMAs. At the top of iteration kt the reads of tile kt are
        // in flight; the wait for them comes before the barrier, so after it
        // every wave is done with the buffer the new DMA refills (tile
        // kt - 1's).
        floatx4 fa[2][P * TM], fb[2][P * TN];
        if (nk >= STAGES - 1)  // the prologue issued STAGES - 1 tiles
            wait_vmcnt<PER_WAVE * (STAGES - 2)>();
        else
            wait_vmcnt<0>();
        __builtin_amdgcn_s_barrier();
        read_group(lds, 0, fa[0], fb[0]);
        auto step = [&](int kt, floatx4 (&ca)[P * TM], floatx4 (&cb)[P * TN], floatx4 (&na)[P * TM],
                        floatx4 (&nb)[P * TN]) {
            lds_wait(ca, cb);
            if (kt + STAGES - 2 < nk)
                wait_vmcnt<PER_WAVE * (STAGES - 3)>();
            else
                wait_vmcnt<0>();
            __builtin_amdgcn_s_barrier();
            if (kt + STAGES - 1 < nk) issue((kt + STAGES - 1) % STAGES, (kt + STAGES - 1) * BK);
            if (kt + 1 < nk) read_group(lds + ((kt + 1) % STAGES) * STAGE, 0, na, nb);
            pin_regs(ca, cb);
            mfma_group(ca, cb);
            __builtin_amdgcn_sched_barrier(0);
        };
        int kt = 0;
        for (; kt + 1 < nk; kt += 2) {
            step(kt, fa[0], fb[0], fa[1], fb[1]);
            step(kt + 1, fa[1], fb[1], fa[0], fb[0]);
        }
        if (kt < nk) step(kt, fa[0], fb[0], fa[1], fb[1]);
    }

    if (m0 + BM <= M && n0 + BN <= N) {
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

// Launches gemm_planes_kernel: K a positive multiple of BK, every plane row
// 16-byte aligned (ld, batch and plane strides multiples of 8 bf16).
template <int BM, int BN, int WAVES_M, int STAGES, int P, int BK, int NW = 4, class EP>
void launch_gemm_planes(hipStream_t stream, int M, int N, int K, int batches, const PlaneRows &al,
                        const PlaneRows &bl, const EP &ep) {
    if (M <= 0 || N <= 0 || batches <= 0) return;
    DMX_REQUIRE(K % BK == 0 && K > 0, "gemm_planes: K must be a positive multiple of the k-tile");
    DMX_REQUIRE(al.ld % 8 == 0 && bl.ld % 8 == 0 && al.plane_stride % 8 == 0 && bl.plane_stride % 8 == 0 &&
                    al.batch_stride % 8 == 0 && bl.batch_stride % 8 == 0 && (uintptr_t)al.p % 16 == 0 &&
                    (uintptr_t)bl.p % 16 == 0,
                "gemm_planes: plane rows must be 16-byte aligned");
    constexpr size_t lds = (size_t)STAGES * P * (BM + BN) * BK * sizeof(unsigned short);
    auto kernel = gemm_planes_kernel<BM, BN, WAVES_M, STAGES, P, BK, NW, EP>;
    static const bool lds_ok = hipFuncSetAttribute(reinterpret_cast<const void *>(kernel),
                                                   hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) == hipSuccess;
    DMX_REQUIRE(lds_ok, "gemm_planes: the kernel's LDS limit could not be raised");
    dim3 grid((unsigned)ceil_div(N, BN), (unsigned)ceil_div(M, BM), (unsigned)batches);
    DMX_REQUIRE(grid.y <= 65535 && grid.z <= 65535, "GEMM grid too large");
    hipLaunchKernelGGL(kernel, grid, dim3(64 * NW), lds, stream, M, N, K, al, bl, ep);
    DMX_LAUNCH_CHECK();
}

}  // namespace dmx
