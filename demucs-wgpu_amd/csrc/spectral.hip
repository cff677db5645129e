// spectral.hip — HTDemucs' STFT front end and iSTFT back end.
//
// Front (crates/demucs-core/src/demucs/spec.rs:62-113, dsp/stft.rs:126-201,
// demucs/host.rs:245-261): reflect pad (1536 | 1536 + le*hop - L), torch.stft
// (center, reflect, periodic Hann, normalized), drop Nyquist and the two pad
// frames each side, CaC packing, per-batch mean / unbiased std of both
// branches, (x - mean) / (1e-5 + std).
// Back (host.rs:465-519, spec.rs:117-175, 268-340, stft.rs:204-295):
// denormalise, CaC unpack, irfft * sqrt(N)/N * window, overlap-add divided by
// the summed squared window, trim, denormalised time branch + the iSTFT.
//
// Only the le kept frames are ever transformed: every sample they read lies
// inside the reflect-padded signal, so the centre padding is never touched,
// and the four zero frames of the inverse only add window energy.
#include <algorithm>

#include "common.h"
#include "ops.h"

namespace dmx {
namespace {

constexpr int FFT_N = 4096;
constexpr int FFT_THREADS = 256;

// 4096-point FFT as three radix-16 Stockham passes (N = 16^3), one thread
// per 16 points (FFT_N / 16 = FFT_THREADS): pass p takes x[j + 256 r],
// r < 16, twiddles it by W^(r (j mod Ns) N / (16 Ns)) (Ns = 16^p), runs a
// 16-point DFT in registers and stores it at (j / Ns) 16 Ns + j mod Ns + r Ns.
// The first pass reads its inputs from the caller and the last pass leaves
// x[j + 256 r] = X[j + 256 r] in registers, so only two exchanges go through
// LDS. W = exp(-2 pi i / N); the inverse (INV) conjugates every twiddle.
constexpr int FFT_R = 16;
static_assert(FFT_N == FFT_R * FFT_R * FFT_R && FFT_N / FFT_R == FFT_THREADS, "radix-16 layout");

__device__ __forceinline__ float2 cadd(float2 a, float2 b) { return make_float2(a.x + b.x, a.y + b.y); }
__device__ __forceinline__ float2 csub(float2 a, float2 b) { return make_float2(a.x - b.x, a.y - b.y); }
__device__ __forceinline__ float2 cmul(float2 a, float2 b) {
    return make_float2(a.x * b.x - a.y * b.y, a.x * b.y + a.y * b.x);
}

// 4-point DFT in place (x0..x3 -> X0..X3); W4 = -i, or +i for the inverse.
template <bool INV>
__device__ __forceinline__ void dft4(float2 &a, float2 &b, float2 &c, float2 &d) {
    const float2 s02 = cadd(a, c), d02 = csub(a, c), s13 = cadd(b, d), d13 = csub(b, d);
    const float2 rot = INV ? make_float2(-d13.y, d13.x) : make_float2(d13.y, -d13.x);  // W4 * d13
    a = cadd(s02, s13);
    c = csub(s02, s13);
    b = cadd(d02, rot);
    d = csub(d02, rot);
}

// 16-point DFT in place, natural order in and out: n = 4 n1 + n2, k = k1 + 4 k2;
// DFT4 over n1, twiddle W16^(n2 k1), DFT4 over n2, then the 4x4 index transpose.
template <bool INV>
__device__ __forceinline__ void dft16(float2 v[16]) {
    constexpr float C1 = 0.92387953251128674f, S1 = 0.38268343236508977f, R2 = 0.70710678118654752f;
    const float sg = INV ? 1.0f : -1.0f;  // sign of the twiddles' imaginary parts
#pragma unroll
    for (int n2 = 0; n2 < 4; ++n2) dft4<INV>(v[n2], v[4 + n2], v[8 + n2], v[12 + n2]);
    // v[4 k1 + n2] *= W16^(n2 k1) for n2, k1 in 1..3 (exponents 1, 2, 3, 2, 4, 6, 3, 6, 9).
    v[5] = cmul(v[5], make_float2(C1, sg * S1));
    v[6] = cmul(v[6], make_float2(R2, sg * R2));
    v[7] = cmul(v[7], make_float2(S1, sg * C1));
    v[9] = cmul(v[9], make_float2(R2, sg * R2));
    v[10] = make_float2(-sg * v[10].y, sg * v[10].x);  // W16^4 = -i (forward)
    v[11] = cmul(v[11], make_float2(-R2, sg * R2));
    v[13] = cmul(v[13], make_float2(S1, sg * C1));
    v[14] = cmul(v[14], make_float2(-R2, sg * R2));
    v[15] = cmul(v[15], make_float2(-C1, -sg * S1));
#pragma unroll
    for (int k1 = 0; k1 < 4; ++k1) dft4<INV>(v[4 * k1], v[4 * k1 + 1], v[4 * k1 + 2], v[4 * k1 + 3]);
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = a + 1; b < 4; ++b) {
            const float2 t = v[4 * a + b];
            v[4 * a + b] = v[4 * b + a];
            v[4 * b + a] = t;
        }
}

// W^e for 0 <= e < N from the half table tw[k] = W^k, k < N/2 (W^(k + N/2) = -W^k).
template <bool INV>
__device__ __forceinline__ float2 twiddle(const float2 *__restrict__ tw, int e) {
    float2 w = tw[e & (FFT_N / 2 - 1)];
    if (e & (FFT_N / 2)) w = make_float2(-w.x, -w.y);
    if (INV) w.y = -w.y;
    return w;
}

// LDS index with one float2 of padding per 16 (the first pass stores with a
// stride of 16 points).
__device__ __forceinline__ int fft_pad(int i) { return i + (i >> 4); }
constexpr int FFT_LDS = FFT_N + FFT_N / 16;

// v[r] = x[j + 256 r] on entry, X[j + 256 r] on exit; `buf` is FFT_LDS float2.
template <bool INV>
__device__ __forceinline__ void fft4096(float2 v[16], float2 *buf, const float2 *__restrict__ tw) {
    const int j = threadIdx.x;
    // pass 0 (Ns = 1): no twiddles; stored at 16 j + r.
    dft16<INV>(v);
#pragma unroll
    for (int r = 0; r < 16; ++r) buf[fft_pad(16 * j + r)] = v[r];
    __syncthreads();
    // pass 1 (Ns = 16): twiddle W^(16 r (j mod 16)); stored at (j / 16) 256 + j mod 16 + 16 r.
#pragma unroll
    for (int r = 0; r < 16; ++r) v[r] = buf[fft_pad(j + 256 * r)];
    {
        const int k = j & 15;
#pragma unroll
        for (int r = 1; r < 16; ++r) v[r] = cmul(v[r], twiddle<INV>(tw, 16 * r * k));
    }
    dft16<INV>(v);
    __syncthreads();
    {
        const int base = (j >> 4) * 256 + (j & 15);
#pragma unroll
        for (int r = 0; r < 16; ++r) buf[fft_pad(base + 16 * r)] = v[r];
    }
    __syncthreads();
    // pass 2 (Ns = 256): twiddle W^(r j); the result stays in registers.
#pragma unroll
    for (int r = 0; r < 16; ++r) v[r] = buf[fft_pad(j + 256 * r)];
#pragma unroll
    for (int r = 1; r < 16; ++r) v[r] = cmul(v[r], twiddle<INV>(tw, r * j));
    dft16<INV>(v);
}

// Reflect index of `pad1d_reflect` (spec.rs:204-236) for inputs longer than the pad.
__device__ __forceinline__ int64_t reflect(int64_t i, int64_t n) {
    if (i < 0) i = -i;
    if (i >= n) i = 2 * (n - 1) - i;
    return i;
}

// Two kept frames (f, f + 1) of one (batch, channel) row per block, as the
// real and imaginary parts of one complex FFT: with z = x1 + i x2,
// X1[k] = (Z[k] + conj Z[N - k]) / 2 and X2[k] = (Z[k] - conj Z[N - k]) / 2i.
// frames_out[row][f][bin] (float2), bins 0..N/2-1, scaled by 1/sqrt(N).
__global__ __launch_bounds__(FFT_THREADS) void stft_kernel(const float *__restrict__ mix, int64_t L, int le,
                                                           const float2 *__restrict__ tw,
                                                           const float *__restrict__ window,
                                                           float2 *__restrict__ frames_out) {
    __shared__ float2 buf[FFT_LDS];
    const int f = 2 * blockIdx.x, row = blockIdx.y, j = threadIdx.x;
    const bool second = f + 1 < le;
    const int hop = FFT_N / 4, pad = hop / 2 * 3;
    const float *x = mix + (int64_t)row * L;
    // Frame f + 2 of the centre-padded signal starts at (f + 2) * hop - N/2 in
    // the reflect-padded one; every index lies inside the padded signal.
    const int64_t start = (int64_t)(f + 2) * hop - FFT_N / 2 - pad;
    float2 v[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int i = j + 256 * r;
        const float w = window[i];
        const float a = x[reflect(start + i, L)];
        const float b = second ? x[reflect(start + hop + i, L)] : 0.0f;
        v[r] = make_float2(a * w, b * w);
    }
    fft4096<false>(v, buf, tw);
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 16; ++r) buf[fft_pad(j + 256 * r)] = v[r];
    __syncthreads();
    const float half_scale = 0.5f / 64.0f;  // the split's 1/2 and 1/sqrt(4096)
    float2 *d1 = frames_out + ((int64_t)row * le + f) * (FFT_N / 2), *d2 = d1 + FFT_N / 2;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
        const int k = j + 256 * r;
        const float2 a = v[r], b = buf[fft_pad((FFT_N - k) & (FFT_N - 1))];  // Z[k], Z[N - k]
        d1[k] = make_float2((a.x + b.x) * half_scale, (a.y - b.y) * half_scale);
        if (second) d2[k] = make_float2((a.y + b.y) * half_scale, (b.x - a.x) * half_scale);
    }
}

// f64 (sum, sum of squares) over `len` floats per batch row blockIdx.y,
// added into stats[stats_stride * row]. VEC: len a multiple of 4 and rows
// 16-byte aligned, read as float4.
template <bool VEC>
__global__ __launch_bounds__(256) void batch_moments_kernel(const float *__restrict__ x, int64_t len,
                                                            double *__restrict__ stats, int stats_stride) {
    const float *row = x + (int64_t)blockIdx.y * len;
    double s = 0.0, q = 0.0;
    if constexpr (VEC) {
        const float4 *p = reinterpret_cast<const float4 *>(row);
        for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < len / 4; i += (int64_t)gridDim.x * 256) {
            const float4 v = p[i];
            const double a = v.x, b = v.y, c = v.z, d = v.w;
            s += (a + b) + (c + d);
            q += (a * a + b * b) + (c * c + d * d);
        }
    } else {
        for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < len; i += (int64_t)gridDim.x * 256) {
            const double v = row[i];
            s += v;
            q += v * v;
        }
    }
    block_moments_atomic(s, q, stats + (int64_t)stats_stride * blockIdx.y);
}

// Moments of b rows of len floats in one launch (grid.y = row).
void batch_moments(hipStream_t s, const float *x, int b, int64_t len, double *stats, int stats_stride) {
    const unsigned per_row = (unsigned)std::max<int64_t>(1, std::min<int64_t>(2048 / std::max(b, 1), 256));
    const bool vec = len % 4 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0;
    if (vec)
        hipLaunchKernelGGL(batch_moments_kernel<true>, dim3(per_row, (unsigned)b), dim3(256), 0, s, x, len, stats,
                           stats_stride);
    else
        hipLaunchKernelGGL(batch_moments_kernel<false>, dim3(per_row, (unsigned)b), dim3(256), 0, s, x, len, stats,
                           stats_stride);
    DMX_LAUNCH_CHECK();
}

// mean and unbiased std per batch (`mean` / `std_unbiased`, demucs/ops.rs:1494-1509, 1585-1590).
__global__ void finish_norms_kernel(const double *__restrict__ stats, int b, double n_spec, double n_wave,
                                    float *__restrict__ norms) {
    int i = threadIdx.x;
    if (i >= b) return;
    const double *sp = stats + 4 * i;
    double m = sp[0] / n_spec, var = (sp[1] - sp[0] * sp[0] / n_spec) / (n_spec - 1.0);
    double mt = sp[2] / n_wave, vart = (sp[3] - sp[2] * sp[2] / n_wave) / (n_wave - 1.0);
    norms[4 * i + 0] = (float)m;
    norms[4 * i + 1] = (float)sqrt(fmax(var, 0.0));
    norms[4 * i + 2] = (float)mt;
    norms[4 * i + 3] = (float)sqrt(fmax(vart, 0.0));
}

// frames (b*2 rows, le, N/2) complex -> xspec (b, 4, N/2, le) normalised CaC:
// channel 2c = re, 2c+1 = im of audio channel c. 32x32 (frame, bin) tiles.
__global__ __launch_bounds__(256) void spec_normalise_kernel(const float2 *__restrict__ frames, int le,
                                                             const float *__restrict__ norms,
                                                             float *__restrict__ xspec) {
    __shared__ float2 tile[32][33];
    const int bins = FFT_N / 2;
    const int row = blockIdx.z, b = row / 2, c = row % 2;
    const int f0 = blockIdx.x * 32, k0 = blockIdx.y * 32;
    const float mean = norms[4 * b], sc = 1.0f / (1e-5f + norms[4 * b + 1]);
    const float2 *src = frames + (int64_t)row * le * bins;
    for (int e = threadIdx.x; e < 32 * 32; e += 256) {
        int fi = e / 32, ki = e % 32, f = f0 + fi;
        tile[fi][ki] = f < le ? src[(int64_t)f * bins + k0 + ki] : make_float2(0.f, 0.f);
    }
    __syncthreads();
    float *re = xspec + ((int64_t)(b * 4 + 2 * c) * bins) * le;
    float *im = re + (int64_t)bins * le;
    for (int e = threadIdx.x; e < 32 * 32; e += 256) {
        int ki = e / 32, fi = e % 32, f = f0 + fi;
        if (f < le) {
            float2 v = tile[fi][ki];
            re[(int64_t)(k0 + ki) * le + f] = (v.x - mean) * sc;
            im[(int64_t)(k0 + ki) * le + f] = (v.y - mean) * sc;
        }
    }
}

__global__ __launch_bounds__(256) void wave_normalise_kernel(const float *__restrict__ mix, int64_t per_batch,
                                                             const float *__restrict__ norms,
                                                             float *__restrict__ out) {
    const int b = blockIdx.y;
    const float mean = norms[4 * b + 2], sc = 1.0f / (1e-5f + norms[4 * b + 3]);
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < per_batch; i += (int64_t)gridDim.x * 256)
        out[b * per_batch + i] = (mix[b * per_batch + i] - mean) * sc;
}

// Denormalise the CaC output (host.rs:466-469: (x + mean/std) * std) and unpack
// to complex frame-major rows: z[(b*S + s)*2 + c][f][bin].
__global__ __launch_bounds__(256) void ispec_prep_kernel(const float *__restrict__ xspec, int S, int le,
                                                         const float *__restrict__ norms, float2 *__restrict__ z) {
    __shared__ float2 tile[32][33];
    const int bins = FFT_N / 2;
    const int row = blockIdx.z, b = row / (2 * S), sc_idx = row % (2 * S), s = sc_idx / 2, c = sc_idx % 2;
    const int k0 = blockIdx.x * 32, f0 = blockIdx.y * 32;
    const float stdv = norms[4 * b + 1], off = -norms[4 * b] / stdv;
    const float *re = xspec + ((int64_t)(b * 4 * S + s * 4 + c * 2) * bins) * le;
    const float *im = re + (int64_t)bins * le;
    for (int e = threadIdx.x; e < 32 * 32; e += 256) {
        int ki = e / 32, fi = e % 32, f = f0 + fi;
        if (f < le) {
            int64_t at = (int64_t)(k0 + ki) * le + f;
            tile[ki][fi] = make_float2((re[at] - off) * stdv, (im[at] - off) * stdv);
        }
    }
    __syncthreads();
    float2 *dst = z + (int64_t)row * le * bins;
    for (int e = threadIdx.x; e < 32 * 32; e += 256) {
        int fi = e / 32, ki = e % 32, f = f0 + fi;
        if (f < le) dst[(int64_t)f * bins + k0 + ki] = tile[ki][fi];
    }
}

// irfft of two kept frames (f, f + 1) per block: Hermitian extensions X1, X2
// (Nyquist = 0, Im X[0] dropped) packed as Z = X1 + i X2, one inverse FFT, real part -> frame
// f and imaginary part -> frame f + 1, each * (sqrt(N)/N) * window ->
// frames_out[row][f][0..N).
__global__ __launch_bounds__(FFT_THREADS) void irfft_kernel(const float2 *__restrict__ z, int le,
                                                            const float2 *__restrict__ tw,
                                                            const float *__restrict__ window,
                                                            float *__restrict__ frames_out) {
    __shared__ float2 buf[FFT_LDS];
    const int f = 2 * blockIdx.x, row = blockIdx.y, j = threadIdx.x;
    const bool second = f + 1 < le;
    const int bins = FFT_N / 2;
    const float2 *s1 = z + ((int64_t)row * le + f) * bins, *s2 = second ? s1 + bins : s1;
    float2 v[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int k = j + 256 * r;
        float2 x1, x2;
        if (r < 8) {
            x1 = s1[k];
            x2 = s2[k];
            if (k == 0) {  // the real part of the inverse ignores Im X[0]; packed, it would leak across
                x1.y = 0.0f;
                x2.y = 0.0f;
            }
        } else {  // k >= N/2: conj X[N - k], zero at the Nyquist bin
            const int m = FFT_N - k;
            const float nz = k == bins ? 0.0f : 1.0f;
            const float2 u1 = s1[m & (bins - 1)], u2 = s2[m & (bins - 1)];
            x1 = make_float2(u1.x * nz, -u1.y * nz);
            x2 = make_float2(u2.x * nz, -u2.y * nz);
        }
        if (!second) x2 = make_float2(0.0f, 0.0f);
        v[r] = make_float2(x1.x - x2.y, x1.y + x2.x);
    }
    fft4096<true>(v, buf, tw);
    const float inv_n = 64.0f / 4096.0f;
    float *d1 = frames_out + ((int64_t)row * le + f) * FFT_N, *d2 = d1 + FFT_N;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int i = j + 256 * r;
        const float w = window[i] * inv_n;
        d1[i] = v[r].x * w;
        if (second) d2[i] = v[r].y * w;
    }
}

// Overlap-add + envelope divide + trim, then out = denorm(time) + wave
// (host.rs:499-512). Output sample n of row r sits at index n + N/2 + pad of
// the iSTFT buffer; frames are added in ascending order as the reference does.
__global__ __launch_bounds__(256) void ola_sum_kernel(const float *__restrict__ frames, int le, int64_t L, int S,
                                                      const float *__restrict__ window,
                                                      const float *__restrict__ xtime,
                                                      const float *__restrict__ norms, float *__restrict__ stems) {
    const int row = blockIdx.y, b = row / (2 * S);
    const int hop = FFT_N / 4, pad = hop / 2 * 3;
    const int total_frames = le + 4;
    const float stdt = norms[4 * b + 3], offt = -norms[4 * b + 2] / stdt;
    const float *fr = frames + (int64_t)row * le * FFT_N;
    for (int64_t n = (int64_t)blockIdx.x * 256 + threadIdx.x; n < L; n += (int64_t)gridDim.x * 256) {
        int64_t i = n + FFT_N / 2 + pad;
        int64_t flo = i >= FFT_N ? (i - FFT_N) / hop + 1 : 0;
        int64_t fhi = i / hop;
        if (fhi > total_frames - 1) fhi = total_frames - 1;
        float y = 0.0f, env = 0.0f;
        for (int64_t F = flo; F <= fhi; ++F) {
            int off = (int)(i - F * hop);
            float w = window[off];
            if (F >= 2 && F < le + 2) y += fr[(F - 2) * FFT_N + off];
            env += w * w;
        }
        float wave = env != 0.0f ? y / env : 0.0f;
        int64_t at = (int64_t)row * L + n;
        float t = (xtime[at] - offt) * stdt;
        stems[at] = t + wave;
    }
}

unsigned grid_cap(int64_t n, int64_t cap) { return (unsigned)std::max<int64_t>(1, std::min<int64_t>(ceil_div(n, 256), cap)); }

}  // namespace

void make_twiddles(int nfft, float *host_out) {
    for (int k = 0; k < nfft / 2; ++k) {
        double ang = 2.0 * 3.14159265358979323846 * (double)k / (double)nfft;
        host_out[2 * k] = (float)std::cos(ang);
        host_out[2 * k + 1] = (float)-std::sin(ang);
    }
    // The periodic Hann window follows the twiddles: (0.5 - 0.5 cos(2 pi i / N)),
    // evaluated in f64 and rounded (crates/demucs-core/src/dsp/stft.rs:54-61).
    for (int i = 0; i < nfft; ++i) {
        double phase = 2.0 * 3.14159265358979323846 * (double)i / (double)nfft;
        host_out[nfft + i] = (float)(0.5 - 0.5 * std::cos(phase));
    }
}

void stft_cac_raw(hipStream_t s, const float *mix, int b, int L, int nfft, float *frames_out, float *xspec_out,
                  const float *twiddles) {
    require_ptrs({mix, frames_out, twiddles}, "stft");
    DMX_REQUIRE(nfft == FFT_N, "stft: only nfft = 4096 is implemented");
    const int hop = nfft / 4, le = (int)ceil_div(L, hop), pad = hop / 2 * 3;
    DMX_REQUIRE(L > pad + le * hop - L && L > pad, "stft: input shorter than the reflect padding");
    const float2 *tw = reinterpret_cast<const float2 *>(twiddles);
    const float *window = twiddles + nfft;
    hipLaunchKernelGGL(stft_kernel, dim3((unsigned)ceil_div(le, 2), (unsigned)(b * 2)), dim3(FFT_THREADS), 0, s, mix, (int64_t)L,
                       le, tw, window, reinterpret_cast<float2 *>(frames_out));
    DMX_LAUNCH_CHECK();
    (void)xspec_out;
}

void spec_and_normalise(hipStream_t s, const float *mix, int b, int L, int nfft, float *frames, float *xspec,
                        float *xwave, float *norms, double *stats, const float *twiddles) {
    require_ptrs({xspec, xwave, norms, stats}, "spec_and_normalise");
    stft_cac_raw(s, mix, b, L, nfft, frames, nullptr, twiddles);
    const int le = (int)ceil_div(L, nfft / 4), bins = nfft / 2;
    // stats layout per batch: (sum, sumsq) spectrum, then (sum, sumsq) wave.
    zero_doubles(s, stats, 4 * (int64_t)b);
    const int64_t spec_len = (int64_t)2 * le * bins * 2;  // 2 channels x le x bins x (re, im)
    DMX_REQUIRE(b <= 1024, "spec_and_normalise: batch too large");
    // One launch per tensor for all batch rows.
    batch_moments(s, frames, b, spec_len, stats, 4);
    batch_moments(s, mix, b, 2 * (int64_t)L, stats + 2, 4);
    hipLaunchKernelGGL(finish_norms_kernel, dim3(1), dim3(1024), 0, s, stats, b, (double)spec_len, 2.0 * L, norms);
    DMX_LAUNCH_CHECK();
    hipLaunchKernelGGL(spec_normalise_kernel, dim3((unsigned)ceil_div(le, 32), (unsigned)(bins / 32), (unsigned)(b * 2)),
                       dim3(256), 0, s, reinterpret_cast<const float2 *>(frames), le, norms, xspec);
    DMX_LAUNCH_CHECK();
    hipLaunchKernelGGL(wave_normalise_kernel, dim3(grid_cap(2 * (int64_t)L, 2048), (unsigned)b), dim3(256), 0, s, mix,
                       2 * (int64_t)L, norms, xwave);
    DMX_LAUNCH_CHECK();
}

void ispec_and_sum(hipStream_t s, const float *xspec, const float *xtime, int b, int S, int L, int nfft, int le,
                   const float *norms, float *frames_scratch, float *stems, const float *twiddles) {
    require_ptrs({xspec, xtime, norms, frames_scratch, stems, twiddles}, "istft");
    DMX_REQUIRE(nfft == FFT_N, "istft: only nfft = 4096 is implemented");
    const int bins = nfft / 2, rows = b * S * 2;
    const float2 *tw = reinterpret_cast<const float2 *>(twiddles);
    const float *window = twiddles + nfft;
    // z (rows, le, bins) complex, then the frames (rows, le, nfft) real, share the scratch:
    // the complex rows sit after the real frames.
    float *frames = frames_scratch;
    float2 *z = reinterpret_cast<float2 *>(frames_scratch + (int64_t)rows * le * nfft);
    hipLaunchKernelGGL(ispec_prep_kernel, dim3((unsigned)(bins / 32), (unsigned)ceil_div(le, 32), (unsigned)rows),
                       dim3(256), 0, s, xspec, S, le, norms, z);
    DMX_LAUNCH_CHECK();
    hipLaunchKernelGGL(irfft_kernel, dim3((unsigned)ceil_div(le, 2), (unsigned)rows), dim3(FFT_THREADS), 0, s, z, le, tw, window,
                       frames);
    DMX_LAUNCH_CHECK();
    hipLaunchKernelGGL(ola_sum_kernel, dim3(grid_cap(L, 512), (unsigned)rows), dim3(256), 0, s, frames, le, (int64_t)L,
                       S, window, xtime, norms, stems);
    DMX_LAUNCH_CHECK();
}

}  // namespace dmx
