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

__device__ __forceinline__ unsigned bitrev12(unsigned i) { return __brev(i) >> 20; }

// In-place radix-2 DIT over buf[FFT_N] already in bit-reversed order.
// tw[k] = exp(-2 pi i k / N), k < N/2; the inverse conjugates it.
__device__ void fft4096(float2 *buf, const float2 *__restrict__ tw, bool inverse) {
    for (int len = 2; len <= FFT_N; len <<= 1) {
        const int half = len >> 1, step = FFT_N / len;
        for (int bf = threadIdx.x; bf < FFT_N / 2; bf += FFT_THREADS) {
            int grp = bf / half, jj = bf - grp * half;
            int i0 = grp * len + jj, i1 = i0 + half;
            float2 w = tw[jj * step];
            if (inverse) w.y = -w.y;
            float2 a = buf[i0], b = buf[i1];
            float2 t = make_float2(b.x * w.x - b.y * w.y, b.x * w.y + b.y * w.x);
            buf[i0] = make_float2(a.x + t.x, a.y + t.y);
            buf[i1] = make_float2(a.x - t.x, a.y - t.y);
        }
        __syncthreads();
    }
}

// Reflect index of `pad1d_reflect` (spec.rs:204-236) for inputs longer than the pad.
__device__ __forceinline__ int64_t reflect(int64_t i, int64_t n) {
    if (i < 0) i = -i;
    if (i >= n) i = 2 * (n - 1) - i;
    return i;
}

// One kept frame of one (batch, channel) row: frames_out[row][f][bin] (float2),
// bins 0..N/2-1, scaled by 1/sqrt(N).
__global__ __launch_bounds__(FFT_THREADS) void stft_kernel(const float *__restrict__ mix, int64_t L, int le,
                                                           const float2 *__restrict__ tw,
                                                           const float *__restrict__ window,
                                                           float2 *__restrict__ frames_out) {
    __shared__ float2 buf[FFT_N];
    const int f = blockIdx.x, row = blockIdx.y;
    const int hop = FFT_N / 4, pad = hop / 2 * 3;
    const int64_t padded_len = (int64_t)le * hop + 2 * pad;
    const float *x = mix + (int64_t)row * L;
    // Frame f + 2 of the centre-padded signal starts at (f + 2) * hop - N/2 in the
    // reflect-padded one.
    const int64_t start = (int64_t)(f + 2) * hop - FFT_N / 2;
    for (int i = threadIdx.x; i < FFT_N; i += FFT_THREADS) {
        int64_t q = start + i;  // in [0, padded_len)
        (void)padded_len;
        int64_t r = reflect(q - pad, L);
        buf[bitrev12(i)] = make_float2(x[r] * window[i], 0.0f);
    }
    __syncthreads();
    fft4096(buf, tw, false);
    const float scale = 1.0f / 64.0f;  // 1/sqrt(4096)
    float2 *dst = frames_out + ((int64_t)row * le + f) * (FFT_N / 2);
    for (int k = threadIdx.x; k < FFT_N / 2; k += FFT_THREADS) {
        float2 v = buf[k];
        dst[k] = make_float2(v.x * scale, v.y * scale);
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

// irfft of one kept frame: Hermitian extension (Nyquist = 0), inverse FFT,
// real part * (sqrt(N)/N) * window -> frames_out[row][f][0..N).
__global__ __launch_bounds__(FFT_THREADS) void irfft_kernel(const float2 *__restrict__ z, int le,
                                                            const float2 *__restrict__ tw,
                                                            const float *__restrict__ window,
                                                            float *__restrict__ frames_out) {
    __shared__ float2 buf[FFT_N];
    const int f = blockIdx.x, row = blockIdx.y;
    const int bins = FFT_N / 2;
    const float2 *src = z + ((int64_t)row * le + f) * bins;
    for (int k = threadIdx.x; k < FFT_N; k += FFT_THREADS) {
        float2 v;
        if (k < bins)
            v = src[k];
        else if (k == bins)
            v = make_float2(0.f, 0.f);
        else {
            float2 u = src[FFT_N - k];
            v = make_float2(u.x, -u.y);
        }
        buf[bitrev12(k)] = v;
    }
    __syncthreads();
    fft4096(buf, tw, true);
    const float inv_n = 64.0f / 4096.0f;
    float *dst = frames_out + ((int64_t)row * le + f) * FFT_N;
    for (int i = threadIdx.x; i < FFT_N; i += FFT_THREADS) dst[i] = buf[i].x * inv_n * window[i];
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
    hipLaunchKernelGGL(stft_kernel, dim3((unsigned)le, (unsigned)(b * 2)), dim3(FFT_THREADS), 0, s, mix, (int64_t)L,
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
    hipLaunchKernelGGL(irfft_kernel, dim3((unsigned)le, (unsigned)rows), dim3(FFT_THREADS), 0, s, z, le, tw, window,
                       frames);
    DMX_LAUNCH_CHECK();
    hipLaunchKernelGGL(ola_sum_kernel, dim3(grid_cap(L, 512), (unsigned)rows), dim3(256), 0, s, frames, le, (int64_t)L,
                       S, window, xtime, norms, stems);
    DMX_LAUNCH_CHECK();
}

}  // namespace dmx
