// winograd.hip — the frequency decoder's 3x3 rewrite (conv2d 3x3, padding 1,
// ic -> 2C channels (ic = C there), on x + skip, then GLU; host.rs:682-759) with Winograd's
// minimal filtering F(2x2, 3x3) (Lavin & Gray, "Fast Algorithms for
// Convolutional Neural Networks", 2016):
//   Y = A^T [ (G g G^T) .* (B^T d B) ] A
// for each 2x2 output tile, with d the 4x4 input patch around it. The
// element-wise product summed over input channels is 16 independent GEMMs,
// one per transformed position xi:  M[xi] (2C x N) = U[xi] (2C x ic) . V[xi]^T,
// N = the 2x2 tiles of all batch rows. Per output that is 16 products per
// four outputs instead of 36 (2.25x fewer MFMA flops).
//   1. wino_input_kernel:  V[xi][n][c] = (B^T (x + skip)_patch B)[xi]
//   2. the direct-to-LDS linear GEMM (both operands k-major), 16 batches
//   3. wino_output_kernel: A^T M A + bias, GLU, into (B, C, F, T)
// U = G g G^T is made once from the PyTorch weight when the model loads.
// Transform matrices:
//   B^T = [1 0 -1 0; 0 1 1 0; 0 -1 1 0; 0 1 0 -1]
//   G   = [1 0 0; 1/2 1/2 1/2; 1/2 -1/2 1/2; 0 0 1]
//   A^T = [1 1 1 0; 0 1 -1 -1]
#include "common.h"
#include "gemm.h"
#include "ops.h"

namespace dmx {
namespace {

constexpr int WI_TILES = 32;                  // tiles (along T) per input block
constexpr int WI_CH = 32;                     // channels per input block
constexpr int WI_COLS = 2 * WI_TILES + 2;     // input columns a block reads
constexpr int WI_CSTRIDE = 4 * WI_COLS + 1;   // odd channel stride in LDS

// V for tiles [j0, j0 + 32) of tile row i, channels [c0, c0 + 32), batch row b.
__global__ __launch_bounds__(256) void wino_input_kernel(const float *__restrict__ x, const float *__restrict__ skip,
                                                         int ic, int F, int T, int TH, int TW, int64_t N,
                                                         float *__restrict__ V) {
    __shared__ float xs[WI_CH * WI_CSTRIDE];
    const int j0 = blockIdx.x * WI_TILES, i = blockIdx.y;
    const int cblocks = (ic + WI_CH - 1) / WI_CH;
    const int b = blockIdx.z / cblocks, c0 = (blockIdx.z - b * cblocks) * WI_CH;
    const int64_t plane = (int64_t)F * T;
    // (x + skip) rows 2i-1 .. 2i+2, columns 2 j0 - 1 .. 2 j0 + 64; zero outside.
    for (int idx = threadIdx.x; idx < WI_CH * 4 * WI_COLS; idx += 256) {
        const int c = idx / (4 * WI_COLS), rem = idx - c * 4 * WI_COLS, r = rem / WI_COLS, col = rem - r * WI_COLS;
        const int y = 2 * i - 1 + r, t = 2 * j0 - 1 + col;
        float v = 0.0f;
        if (c0 + c < ic && y >= 0 && y < F && t >= 0 && t < T) {
            const int64_t at = ((int64_t)b * ic + c0 + c) * plane + (int64_t)y * T + t;
            v = x[at] + (skip ? skip[at] : 0.0f);
        }
        xs[c * WI_CSTRIDE + r * WI_COLS + col] = v;
    }
    __syncthreads();
    // Lane -> channel (consecutive lanes write consecutive channels of a row of V).
    const int c = threadIdx.x % WI_CH, tg = threadIdx.x / WI_CH;
    if (c0 + c >= ic) return;
    const float *p = xs + c * WI_CSTRIDE;
#pragma unroll
    for (int k = 0; k < WI_TILES / 8; ++k) {
        const int jj = tg * (WI_TILES / 8) + k, j = j0 + jj;
        if (j >= TW) break;
        float d[4][4];
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int q = 0; q < 4; ++q) d[r][q] = p[r * WI_COLS + 2 * jj + q];
        float t[4][4];  // B^T d
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            t[0][q] = d[0][q] - d[2][q];
            t[1][q] = d[1][q] + d[2][q];
            t[2][q] = d[2][q] - d[1][q];
            t[3][q] = d[1][q] - d[3][q];
        }
        const int64_t n = ((int64_t)b * TH + i) * TW + j;
        float *dst = V + n * ic + c0 + c;
        const int64_t xi_stride = N * ic;
#pragma unroll
        for (int r = 0; r < 4; ++r) {  // (B^T d) B, row r
            dst[(4 * r + 0) * xi_stride] = t[r][0] - t[r][2];
            dst[(4 * r + 1) * xi_stride] = t[r][1] + t[r][2];
            dst[(4 * r + 2) * xi_stride] = t[r][2] - t[r][1];
            dst[(4 * r + 3) * xi_stride] = t[r][1] - t[r][3];
        }
    }
}

// M[xi] rows are the 2C output channels, columns the tiles: a plain store.
struct EpWinoStore {
    float *out;
    int64_t ldo, batch_stride;
    __device__ void init(int) {}
    __device__ void store(int z, int m, int n, float v) { out[z * batch_stride + (int64_t)m * ldo + n] = v; }
    template <int TM, int TN>
    __device__ void store_frags(int z, int mb, int nb, int col, int khalf, const floatx16 (&v)[TM][TN]) {
        float *o = out + z * batch_stride;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    o[(int64_t)(mb + 32 * i + 8 * (r / 4) + 4 * khalf + r % 4) * ldo + nb + 32 * j + col] = v[i][j][r];
    }
    __device__ void finalize(int) {}
};

// Tile n of channel c: Y = A^T M A for the value (c) and gate (C + c) rows,
// bias, GLU, into out (B, C, F, T).
__global__ __launch_bounds__(256) void wino_output_kernel(const float *__restrict__ Mt, int C, int F, int T, int TH,
                                                          int TW, int64_t N, const float *__restrict__ bias,
                                                          float *__restrict__ out) {
    const int64_t n = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int c = blockIdx.y;
    if (n >= N) return;
    const int64_t xi_stride = 2 * (int64_t)C * N;
    float yv[2][2], yg[2][2];
    for (int half = 0; half < 2; ++half) {
        const float *m = Mt + (int64_t)(half ? C + c : c) * N + n;
        float s[2][4];  // A^T M
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float m0 = m[(0 + q) * xi_stride], m1 = m[(4 + q) * xi_stride];
            const float m2 = m[(8 + q) * xi_stride], m3 = m[(12 + q) * xi_stride];
            s[0][q] = m0 + m1 + m2;
            s[1][q] = m1 - m2 - m3;
        }
        float(&y)[2][2] = half ? yg : yv;
#pragma unroll
        for (int a = 0; a < 2; ++a) {  // (A^T M) A
            y[a][0] = s[a][0] + s[a][1] + s[a][2];
            y[a][1] = s[a][1] - s[a][2] - s[a][3];
        }
    }
    const float bv = bias[c], bg = bias[C + c];
    const int j = (int)(n % TW), i = (int)((n / TW) % TH), b = (int)(n / ((int64_t)TW * TH));
    float *o = out + ((int64_t)b * C + c) * F * T;
#pragma unroll
    for (int a = 0; a < 2; ++a) {
        const int y = 2 * i + a;
        if (y >= F) break;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int t = 2 * j + e;
            if (t < T) o[(int64_t)y * T + t] = (yv[a][e] + bv) * sigmoid(yg[a][e] + bg);
        }
    }
}

}  // namespace

#ifndef DMX_WINO_MIN_C
#define DMX_WINO_MIN_C 192  // narrower layers stay direct: their transforms would move more bytes than MFMA saves
#endif
bool winograd_channels(int ic, int C) { return DMX_WINO_MIN_C > 0 && C >= DMX_WINO_MIN_C && ic % 16 == 0; }

bool winograd_applies(int ic, int C, int F, int T) {
    return winograd_channels(ic, C) && F >= 1 && T >= 1 && mfma_precision() == MfmaPrecision::FP32;
}

int64_t winograd_scratch_floats(int B, int ic, int C, int F, int T) {
    const int64_t N = (int64_t)B * ((F + 1) / 2) * ((T + 1) / 2);
    return 16 * N * (int64_t)ic + 16 * N * 2 * (int64_t)C;
}

void winograd_weights(const float *w, int oc, int ic, float *U) {
    // U[xi = 4p + q][o][c] = sum_{u,v} G[p][u] g[u][v] G[q][v]
    static const double G[4][3] = {{1, 0, 0}, {0.5, 0.5, 0.5}, {0.5, -0.5, 0.5}, {0, 0, 1}};
    for (int o = 0; o < oc; ++o)
        for (int c = 0; c < ic; ++c) {
            const float *g = w + ((int64_t)o * ic + c) * 9;
            double gt[4][3];  // G g
            for (int p = 0; p < 4; ++p)
                for (int v = 0; v < 3; ++v) gt[p][v] = G[p][0] * g[v] + G[p][1] * g[3 + v] + G[p][2] * g[6 + v];
            for (int p = 0; p < 4; ++p)
                for (int q = 0; q < 4; ++q)
                    U[((int64_t)(4 * p + q) * oc + o) * ic + c] =
                        (float)(gt[p][0] * G[q][0] + gt[p][1] * G[q][1] + gt[p][2] * G[q][2]);
        }
}

void conv3x3_glu_winograd(hipStream_t s, const float *x, const float *skip, int B, int ic, int C, int F, int T,
                          const float *U, const float *bias, float *out, float *scratch) {
    require_ptrs({x, U, bias, out, scratch}, "conv3x3_glu_winograd");
    DMX_REQUIRE(ic % 16 == 0 && C > 0, "winograd: the input channel count must be a multiple of 16");
    const int TH = (F + 1) / 2, TW = (T + 1) / 2;
    const int64_t N = (int64_t)B * TH * TW;
    DMX_REQUIRE(N <= INT32_MAX && TH <= 65535, "winograd: too many tiles");
    float *V = scratch, *Mt = scratch + 16 * N * ic;
    const int cblocks = (ic + WI_CH - 1) / WI_CH;
    DMX_REQUIRE((int64_t)B * cblocks <= 65535, "winograd: too many batch rows");
    hipLaunchKernelGGL(wino_input_kernel, dim3((unsigned)ceil_div(TW, WI_TILES), (unsigned)TH, (unsigned)(B * cblocks)),
                       dim3(256), 0, s, x, skip, ic, F, T, TH, TW, N, V);
    DMX_LAUNCH_CHECK();
    EpWinoStore ep{Mt, N, 2 * (int64_t)C * N};
    launch_gemm_dma<128, 128, 2, 4>(s, 2 * C, (int)N, ic, 16, KMajorRows{U, ic, 2 * (int64_t)C * ic},
                                    KMajorRows{V, ic, N * ic}, ep);
    hipLaunchKernelGGL(wino_output_kernel, dim3((unsigned)ceil_div(N, 256), (unsigned)C), dim3(256), 0, s, Mt, C, F,
                       T, TH, TW, N, bias, out);
    DMX_LAUNCH_CHECK();
}

}  // namespace dmx
