// winograd.hip — the frequency decoder's 3x3 rewrite (conv2d 3x3, padding 1,
// ic -> 2C channels (ic = C there), on x + skip, then GLU; host.rs:682-759)
// with Winograd's minimal filtering F(m x m, 3 x 3) (Lavin & Gray, "Fast
// Algorithms for Convolutional Neural Networks", 2016), m = 2 or 4:
//   Y = A^T [ (G g G^T) .* (B^T d B) ] A
// for each m x m output tile, with d the (m+2) x (m+2) input patch around it.
// The element-wise product summed over input channels is (m+2)^2 independent
// GEMMs, one per transformed position xi:
//   M[xi] (2C x N) = U[xi] (2C x ic) . V[xi]^T,   N = the tiles of all batch rows,
// i.e. (m+2)^2 products per m^2 outputs instead of 9 m^2: 2.25x fewer MFMA
// flops for m = 2, 4x for m = 4.
//   1. wino_input_kernel:  V[xi][n][c] = (B^T (x + skip)_patch B)[xi]
//   2. the direct-to-LDS linear GEMM (both operands k-major), (m+2)^2 batches
//   3. wino_output_kernel: A^T M A + bias, GLU, into (B, C, F, T)
// U = G g G^T is made once (in f64) from the PyTorch weight when the model loads.
// Transform matrices (interpolation points 0, 1, -1, inf for m = 2;
// 0, 1, -1, 2, -2, inf for m = 4):
//   m = 2: B^T = [1 0 -1 0; 0 1 1 0; 0 -1 1 0; 0 1 0 -1]
//          G   = [1 0 0; 1/2 1/2 1/2; 1/2 -1/2 1/2; 0 0 1]
//          A^T = [1 1 1 0; 0 1 -1 -1]
//   m = 4: B^T = [4 0 -5 0 1 0; 0 -4 -4 1 1 0; 0 4 -4 -1 1 0; 0 -2 -1 2 1 0;
//                 0 2 -1 -2 1 0; 0 4 0 -5 0 1]
//          G   = [1/4 0 0; -1/6 -1/6 -1/6; -1/6 1/6 -1/6; 1/24 1/12 1/6;
//                 1/24 -1/12 1/6; 0 0 1]
//          A^T = [1 1 1 1 1 0; 0 1 -1 2 -2 0; 0 1 1 4 4 0; 0 1 -1 8 -8 1]
#include "common.h"
#include "gemm.h"
#include "ops.h"

namespace dmx {
namespace {

template <int WT>
struct Wino;

template <>
struct Wino<2> {
    __device__ static void bt(const float *d, float *o) {  // B^T d, d of length 4
        o[0] = d[0] - d[2];
        o[1] = d[1] + d[2];
        o[2] = d[2] - d[1];
        o[3] = d[1] - d[3];
    }
    __device__ static void at(const float *m, float *y) {  // A^T m, m of length 4
        y[0] = m[0] + m[1] + m[2];
        y[1] = m[1] - m[2] - m[3];
    }
};

template <>
struct Wino<4> {
    __device__ static void bt(const float *d, float *o) {  // B^T d, d of length 6
        o[0] = fmaf(4.0f, d[0], fmaf(-5.0f, d[2], d[4]));
        o[1] = fmaf(-4.0f, d[1] + d[2], d[3] + d[4]);
        o[2] = fmaf(4.0f, d[1] - d[2], d[4] - d[3]);
        o[3] = fmaf(2.0f, d[3] - d[1], d[4] - d[2]);
        o[4] = fmaf(2.0f, d[1] - d[3], d[4] - d[2]);
        o[5] = fmaf(4.0f, d[1], fmaf(-5.0f, d[3], d[5]));
    }
    __device__ static void at(const float *m, float *y) {  // A^T m, m of length 6
        const float a = m[1] + m[2], b = m[1] - m[2], c = m[3] + m[4], e = m[3] - m[4];
        y[0] = m[0] + a + c;
        y[1] = fmaf(2.0f, e, b);
        y[2] = fmaf(4.0f, c, a);
        y[3] = fmaf(8.0f, e, b) + m[5];
    }
};

constexpr int WI_CH = 32;    // channels per input block
constexpr int WI_COLS = 66;  // input columns a block reads: tiles * m + 2

// V for tiles [j0, j0 + TILES) of tile row i, channels [c0, c0 + 32), batch row b.
template <int WT>
__global__ __launch_bounds__(256) void wino_input_kernel(const float *__restrict__ x, const float *__restrict__ skip,
                                                         int ic, int F, int T, int TH, int TW, int64_t N,
                                                         float *__restrict__ V) {
    constexpr int A = WT + 2, TILES = (WI_COLS - 2) / WT, CSTRIDE = A * WI_COLS + 1;  // odd channel stride
    __shared__ float xs[WI_CH * CSTRIDE];
    const int j0 = blockIdx.x * TILES, i = blockIdx.y;
    const int cblocks = (ic + WI_CH - 1) / WI_CH;
    const int b = blockIdx.z / cblocks, c0 = (blockIdx.z - b * cblocks) * WI_CH;
    const int64_t plane = (int64_t)F * T;
    // (x + skip) rows WT i - 1 .. WT i + WT, columns WT j0 - 1 .. WT j0 + 64; zero outside.
    for (int idx = threadIdx.x; idx < WI_CH * A * WI_COLS; idx += 256) {
        const int c = idx / (A * WI_COLS), rem = idx - c * A * WI_COLS, r = rem / WI_COLS, col = rem - r * WI_COLS;
        const int y = WT * i - 1 + r, t = WT * j0 - 1 + col;
        float v = 0.0f;
        if (c0 + c < ic && y >= 0 && y < F && t >= 0 && t < T) {
            const int64_t at = ((int64_t)b * ic + c0 + c) * plane + (int64_t)y * T + t;
            v = x[at] + (skip ? skip[at] : 0.0f);
        }
        xs[c * CSTRIDE + r * WI_COLS + col] = v;
    }
    __syncthreads();
    // Lane -> channel: consecutive lanes write consecutive channels of a row of V.
    const int c = threadIdx.x % WI_CH, tg = threadIdx.x / WI_CH;
    if (c0 + c >= ic) return;
    const float *p = xs + c * CSTRIDE;
    const int64_t xi_stride = N * ic;
#pragma unroll
    for (int k = 0; k < TILES / 8; ++k) {
        const int jj = tg * (TILES / 8) + k, j = j0 + jj;
        if (j >= TW) break;
        float t[A][A];  // B^T d, column by column
#pragma unroll
        for (int q = 0; q < A; ++q) {
            float col[A], o[A];
#pragma unroll
            for (int r = 0; r < A; ++r) col[r] = p[r * WI_COLS + WT * jj + q];
            Wino<WT>::bt(col, o);
#pragma unroll
            for (int r = 0; r < A; ++r) t[r][q] = o[r];
        }
        float *dst = V + (((int64_t)b * TH + i) * TW + j) * ic + c0 + c;
#pragma unroll
        for (int r = 0; r < A; ++r) {  // (B^T d) B, row r
            float o[A];
            Wino<WT>::bt(t[r], o);
#pragma unroll
            for (int q = 0; q < A; ++q) dst[(A * r + q) * xi_stride] = o[q];
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
template <int WT>
__global__ __launch_bounds__(256) void wino_output_kernel(const float *__restrict__ Mt, int C, int F, int T, int TH,
                                                          int TW, int64_t N, const float *__restrict__ bias,
                                                          float *__restrict__ out) {
    constexpr int A = WT + 2;
    const int64_t n = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int c = blockIdx.y;
    if (n >= N) return;
    const int64_t xi_stride = 2 * (int64_t)C * N;
    float y[2][WT][WT];  // value, gate
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const float *m = Mt + (int64_t)(h ? C + c : c) * N + n;
        float s[WT][A];  // A^T M, column by column
#pragma unroll
        for (int q = 0; q < A; ++q) {
            float col[A], o[WT];
#pragma unroll
            for (int r = 0; r < A; ++r) col[r] = m[(A * r + q) * xi_stride];
            Wino<WT>::at(col, o);
#pragma unroll
            for (int a = 0; a < WT; ++a) s[a][q] = o[a];
        }
#pragma unroll
        for (int a = 0; a < WT; ++a) Wino<WT>::at(s[a], y[h][a]);  // (A^T M) A, row a
    }
    const float bv = bias[c], bg = bias[C + c];
    const int j = (int)(n % TW), i = (int)((n / TW) % TH), b = (int)(n / ((int64_t)TW * TH));
    float *o = out + ((int64_t)b * C + c) * F * T;
#pragma unroll
    for (int a = 0; a < WT; ++a) {
        const int yy = WT * i + a;
        if (yy >= F) break;
#pragma unroll
        for (int e = 0; e < WT; ++e) {
            const int t = WT * j + e;
            if (t < T) o[(int64_t)yy * T + t] = (y[0][a][e] + bv) * sigmoid(y[1][a][e] + bg);
        }
    }
}

// G of F(m x m, 3 x 3): rows of the weight transform.
const double G2[4][3] = {{1, 0, 0}, {0.5, 0.5, 0.5}, {0.5, -0.5, 0.5}, {0, 0, 1}};
const double G4[6][3] = {{0.25, 0, 0},
                         {-1.0 / 6, -1.0 / 6, -1.0 / 6},
                         {-1.0 / 6, 1.0 / 6, -1.0 / 6},
                         {1.0 / 24, 1.0 / 12, 1.0 / 6},
                         {1.0 / 24, -1.0 / 12, 1.0 / 6},
                         {0, 0, 1}};

template <int WT>
void run(hipStream_t s, const float *x, const float *skip, int B, int ic, int C, int F, int T, const float *U,
         const float *bias, float *out, float *scratch) {
    constexpr int A = WT + 2, XI = A * A, TILES = (WI_COLS - 2) / WT;
    const int TH = (F + WT - 1) / WT, TW = (T + WT - 1) / WT;
    const int64_t N = (int64_t)B * TH * TW;
    DMX_REQUIRE(N <= INT32_MAX && TH <= 65535, "winograd: too many tiles");
    float *V = scratch, *Mt = scratch + XI * N * ic;
    const int cblocks = (ic + WI_CH - 1) / WI_CH;
    DMX_REQUIRE((int64_t)B * cblocks <= 65535, "winograd: too many batch rows");
    hipLaunchKernelGGL(wino_input_kernel<WT>, dim3((unsigned)ceil_div(TW, TILES), (unsigned)TH, (unsigned)(B * cblocks)),
                       dim3(256), 0, s, x, skip, ic, F, T, TH, TW, N, V);
    DMX_LAUNCH_CHECK();
    EpWinoStore ep{Mt, N, 2 * (int64_t)C * N};
    launch_gemm_dma<128, 128, 2, 4>(s, 2 * C, (int)N, ic, XI, KMajorRows{U, ic, 2 * (int64_t)C * ic},
                                    KMajorRows{V, ic, N * ic}, ep);
    hipLaunchKernelGGL(wino_output_kernel<WT>, dim3((unsigned)ceil_div(N, 256), (unsigned)C), dim3(256), 0, s, Mt, C,
                       F, T, TH, TW, N, bias, out);
    DMX_LAUNCH_CHECK();
}

}  // namespace

// Output tile m of the layers that take this path (0: none), and the narrowest
// such layer: narrower layers stay direct, where the transforms would move more
// bytes than the MFMA work they save.
#ifndef DMX_WINO_TILE
#define DMX_WINO_TILE 4
#endif
#ifndef DMX_WINO_MIN_C
#define DMX_WINO_MIN_C 96
#endif
static_assert(DMX_WINO_TILE == 0 || DMX_WINO_TILE == 2 || DMX_WINO_TILE == 4, "the Winograd tile is 2 or 4");

int winograd_tile(int ic, int C) { return (DMX_WINO_TILE && C >= DMX_WINO_MIN_C && ic % 16 == 0) ? DMX_WINO_TILE : 0; }

bool winograd_applies(int ic, int C, int F, int T) {
    return winograd_tile(ic, C) && F >= 1 && T >= 1 && !bf16_mfma();
}

int64_t winograd_weight_floats(int ic, int C) {
    const int a = winograd_tile(ic, C) + 2;
    return (int64_t)a * a * 2 * C * ic;
}

int64_t winograd_scratch_floats(int B, int ic, int C, int F, int T) {
    const int wt = winograd_tile(ic, C);
    if (!wt) return 0;
    const int a = wt + 2;
    const int64_t N = (int64_t)B * ((F + wt - 1) / wt) * ((T + wt - 1) / wt);
    return (int64_t)a * a * N * ((int64_t)ic + 2 * (int64_t)C);
}

void winograd_weights(const float *w, int oc, int ic, float *U) {
    // U[xi = A p + q][o][c] = sum_{u,v} G[p][u] g[u][v] G[q][v]
    const int wt = winograd_tile(ic, oc / 2), a = wt + 2;
    DMX_REQUIRE(wt != 0, "winograd_weights: this layer does not take the Winograd path");
    auto Gm = [&](int p, int u) { return wt == 2 ? G2[p][u] : G4[p][u]; };
    for (int o = 0; o < oc; ++o)
        for (int c = 0; c < ic; ++c) {
            const float *g = w + ((int64_t)o * ic + c) * 9;
            double gt[6][3];  // G g
            for (int p = 0; p < a; ++p)
                for (int v = 0; v < 3; ++v) gt[p][v] = Gm(p, 0) * g[v] + Gm(p, 1) * g[3 + v] + Gm(p, 2) * g[6 + v];
            for (int p = 0; p < a; ++p)
                for (int q = 0; q < a; ++q)
                    U[((int64_t)(a * p + q) * oc + o) * ic + c] =
                        (float)(gt[p][0] * Gm(q, 0) + gt[p][1] * Gm(q, 1) + gt[p][2] * Gm(q, 2));
        }
}

void conv3x3_glu_winograd(hipStream_t s, const float *x, const float *skip, int B, int ic, int C, int F, int T,
                          const float *U, const float *bias, float *out, float *scratch) {
    require_ptrs({x, U, bias, out, scratch}, "conv3x3_glu_winograd");
    const int wt = winograd_tile(ic, C);
    DMX_REQUIRE(wt != 0, "conv3x3_glu_winograd: this layer does not take the Winograd path");
    if (wt == 2)
        run<2>(s, x, skip, B, ic, C, F, T, U, bias, out, scratch);
    else
        run<4>(s, x, skip, B, ic, C, F, T, U, bias, out, scratch);
}

}  // namespace dmx
