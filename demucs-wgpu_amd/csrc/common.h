// common.h — shared host/device helpers for the HIP backend (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <stdexcept>
#include <string>

#include "status.h"

namespace dmx {

#define DMX_HIP(expr)                                                                             \
    do {                                                                                          \
        hipError_t _e = (expr);                                                                   \
        if (_e != hipSuccess)                                                                     \
            ::dmx::throw_error(6, std::string(#expr) + " failed: " + hipGetErrorString(_e) +      \
                                      " (" + __FILE__ + ":" + std::to_string(__LINE__) + ")");  \
    } while (0)

#define DMX_LAUNCH_CHECK() DMX_HIP(hipGetLastError())

#define DMX_REQUIRE(cond, msg)                                                                    \
    do {                                                                                          \
        if (!(cond)) ::dmx::throw_error(1, std::string(msg));                                     \
    } while (0)

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Host-side check that every operand a kernel will dereference is non-null,
// so a wiring mistake is an error at the launch instead of a device fault.
inline void require_ptrs(std::initializer_list<const void *> ptrs, const char *what) {
    for (const void *p : ptrs)
        if (!p) throw Error(8, std::string(what) + ": null device pointer");
}


// Input precision of the MFMA contractions (GEMMs, attention) that the
// calling thread launches. The runner sets it per call from its precision;
// accumulation, softmax, norms and outputs are fp32 either way.
// - FP32: every contraction on the fp32 matrix cores.
// - FP32X3: the same, except the transformer linears, which run on the bf16
//   matrix cores over three bf16 planes per operand (gemm_planes.h), an fp32
//   product to fp32 accuracy.
// - BF16: contractions take bf16 inputs (the linears one bf16 plane).
enum class MfmaPrecision { FP32, BF16, FP32X3 };
inline MfmaPrecision &mfma_precision() {
    static thread_local MfmaPrecision p = MfmaPrecision::FP32X3;  // DMX_PRECISION_FP32
    return p;
}
inline bool bf16_mfma() { return mfma_precision() == MfmaPrecision::BF16; }
// bf16 planes per operand of the transformer linears (0: fp32 MFMA).
inline int linear_planes() {
    switch (mfma_precision()) {
        case MfmaPrecision::FP32X3: return 3;
        case MfmaPrecision::BF16: return 1;
        default: return 0;
    }
}
// A dmx_precision value (dmx.h) as the MFMA precision of what it launches.
inline MfmaPrecision mfma_of_precision(int precision) {
    switch (precision) {
        case 0: return MfmaPrecision::FP32X3;  // DMX_PRECISION_FP32
        case 1: return MfmaPrecision::BF16;    // DMX_PRECISION_BF16
        case 2: return MfmaPrecision::FP32;    // DMX_PRECISION_FP32_MFMA
        default: throw Error(8, "unknown precision " + std::to_string(precision));
    }
}
struct MfmaPrecisionScope {
    MfmaPrecision prev;
    explicit MfmaPrecisionScope(MfmaPrecision p) : prev(mfma_precision()) { mfma_precision() = p; }
    ~MfmaPrecisionScope() { mfma_precision() = prev; }
    MfmaPrecisionScope(const MfmaPrecisionScope &) = delete;
    MfmaPrecisionScope &operator=(const MfmaPrecisionScope &) = delete;
};

// ---------------------------------------------------------------------------
// Device math shared by every kernel.
// ---------------------------------------------------------------------------

// erf via the Numerical Recipes rational approximation of erfc (Press et al.,
// "erfcc", fractional error < 1.2e-7) — the same published formula the
// reference's CPU GELU uses (crates/demucs-core/src/ops.rs:101-121). The
// reciprocal and the exponential are the hardware ones (v_rcp_f32,
// v_exp_f32: about 1 ulp each), which keeps the device within a few 1e-7 of
// the formula at a third of the instructions of the IEEE sequences.
__device__ __forceinline__ float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }
__device__ __forceinline__ float erf_nr(float x) {
    float z = fabsf(x);
    float t = __builtin_amdgcn_rcpf(1.0f + 0.5f * z);
    float poly =
        -z * z - 1.26551223f +
        t * (1.00002368f +
             t * (0.37409196f +
                  t * (0.09678418f +
                       t * (-0.18628806f +
                            t * (0.27886807f +
                                 t * (-1.13520398f +
                                      t * (1.48851587f + t * (-0.82215223f + t * 0.17087277f))))))));
    float tau = t * fast_exp(poly);
    float value = 1.0f - tau;
    return x >= 0.0f ? value : -value;
}

// Exact (erf) GELU: 0.5 x (1 + erf(x / sqrt 2)).
__device__ __forceinline__ float gelu(float x) { return 0.5f * x * (1.0f + erf_nr(x * 0.70710678118654752440f)); }

// Logistic sigmoid with the hardware reciprocal and exponential.
__device__ __forceinline__ float sigmoid(float g) { return __builtin_amdgcn_rcpf(1.0f + fast_exp(-g)); }

// Workgroup placement across the 8 XCDs (each with its own L2): blocks are
// handed out round-robin, block i to XCD i % 8. xcd_contiguous() maps the
// launch index to a logical block so that each XCD runs one contiguous range
// of the logical order (sizes differ by at most one), which keeps blocks that
// share operand panels on one L2. DMX_XCD_REMAP=0 keeps the launch order.
#ifndef DMX_XCD_REMAP
#define DMX_XCD_REMAP 1
#endif
constexpr int XCDS = 8;
__device__ __forceinline__ int xcd_contiguous(int bid, int total) {
#if DMX_XCD_REMAP
    const int x = bid % XCDS, local = bid / XCDS, q = total / XCDS, r = total % XCDS;
    return x < r ? x * (q + 1) + local : r * (q + 1) + (x - r) * q + local;
#else
    (void)total;
    return bid;
#endif
}

// bf16 planes of fp32 values: x = x_0 + x_1 + ..., x_q the round-to-nearest-
// even bf16 of what x_0 .. x_{q-1} leave. Each residual is exact in fp32, and
// each plane carries the next 8 significant bits.
__device__ __forceinline__ unsigned short bf16_split_step(float &x) {
    const __bf16 h = (__bf16)x;
    x -= (float)h;
    return __builtin_bit_cast(unsigned short, h);
}
// Two values -> P planes as packed pairs, the same bits as bf16_split_step
// on each: w[q] holds plane q of a0 (low half) and of a1 (high half). One
// v_cvt_pk_bf16_f32 per plane; the residuals take the planes' bits straight
// from the packed pair.
template <int P>
__device__ __forceinline__ void split_pair_planes(float a0, float a1, unsigned (&w)[P]) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    typedef float floatx2_t __attribute__((ext_vector_type(2)));
#pragma unroll
    for (int q = 0; q < P; ++q) {
        const unsigned u = __builtin_bit_cast(unsigned, __builtin_convertvector((floatx2_t){a0, a1}, bf16x2_t));
        w[q] = u;
        if (q + 1 < P) {
            a0 -= __builtin_bit_cast(float, u << 16);
            a1 -= __builtin_bit_cast(float, u & 0xffff0000u);
        }
    }
}
// Four consecutive values -> P planes, 8 bytes per plane at dst + q * stride.
template <int P>
__device__ __forceinline__ void store_planes4(unsigned short *dst, int64_t stride, float4 v) {
    unsigned lo[P], hi[P];
    split_pair_planes<P>(v.x, v.y, lo);
    split_pair_planes<P>(v.z, v.w, hi);
#pragma unroll
    for (int q = 0; q < P; ++q) *reinterpret_cast<uint2 *>(dst + q * stride) = make_uint2(lo[q], hi[q]);
}
// Two values -> P planes, a0's at dst + q * stride and a1's `step` further.
template <int P>
__device__ __forceinline__ void store_planes2(unsigned short *dst, int64_t step, int64_t stride, float a0, float a1) {
    unsigned w[P];
    split_pair_planes<P>(a0, a1, w);
#pragma unroll
    for (int q = 0; q < P; ++q) {
        dst[q * stride] = (unsigned short)w[q];
        dst[q * stride + step] = (unsigned short)(w[q] >> 16);
    }
}
// One value -> P planes.
template <int P>
__device__ __forceinline__ void store_planes1(unsigned short *dst, int64_t stride, float v) {
#pragma unroll
    for (int q = 0; q < P; ++q) dst[q * stride] = bf16_split_step(v);
}

// Wave64 reductions.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// Block-wide f64 (sum, sum of squares) reduction, then one atomic add per block
// into dst[0], dst[1]. blockDim.x must be a multiple of 64 and <= 1024.
__device__ inline void block_moments_atomic(double s, double q, double *dst) {
    __shared__ double red_s[16], red_q[16];
    s = wave_sum_d(s);
    q = wave_sum_d(q);
    int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    if (lane == 0) {
        red_s[wave] = s;
        red_q[wave] = q;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        double ts = 0.0, tq = 0.0;
        for (int w = 0; w < waves; ++w) {
            ts += red_s[w];
            tq += red_q[w];
        }
        atomicAdd(dst, ts);
        atomicAdd(dst + 1, tq);
    }
}

// GroupNorm(1) statistics from (sum, sum of squares) in f64, as the reference
// turns them into f32 (crates/demucs-core/src/demucs/ops.rs:568-579):
// mean = s/n, var = max(q/n - mean^2, 0), inv = 1 / (float)sqrt(var + 1e-5).
__device__ __forceinline__ void gn_stats(const double *sq, double count, float &mean, float &inv) {
    double m = sq[0] / count;
    double var = fmax(sq[1] / count - m * m, 0.0);
    mean = (float)m;
    inv = 1.0f / (float)sqrt(var + 1e-5);
}

}  // namespace dmx
