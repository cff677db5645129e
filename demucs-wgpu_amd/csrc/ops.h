// ops.h — host-side launchers of the HIP kernels. Every launcher enqueues on
// `stream`, validates what the kernel's grid assumes, and never synchronises.
// Device pointers throughout; layouts follow PyTorch (row-major, (b, c, ...)).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace dmx {

enum Act { ACT_NONE = 0, ACT_GELU = 1 };

// ---------------- GEMM-based ops (conv.hip, gemm.h) ----------------

// Convolution weights in GEMM order. A PyTorch (oc, ic, kh, kw) weight is
// consumed in channel quads whenever conv_tap_major(ic, kh, kw): the
// implicit-GEMM k index is (c / 4 * taps + tap) * 4 + c % 4, i.e. the weight
// is read as (oc, ic / 4, kh * kw, 4). Four consecutive k are then four
// channels at one tap (one bounds test per four loads), and the taps of a
// quad follow each other, so a k-tile re-reads input rows the previous one
// just fetched. Otherwise the PyTorch layout is used as is.
// conv_gemm_weights() makes the GEMM-order copy (host arrays).
inline bool conv_tap_major(int ic, int kh, int kw) { return kh * kw > 1 && ic % 4 == 0; }
void conv_gemm_weights(const float *w, int oc, int ic, int kh, int kw, float *out);

// nn.Conv2d over (b, ic, h, w): weight (oc, ic, kh, kw) in GEMM order (above),
// optional bias; act on output.
// `skip` (same shape as x, may be null) is added to the input while it is gathered.
void conv2d(hipStream_t s, const float *x, const float *skip, int b, int ic, int h, int w, const float *weight,
            const float *bias, int oc, int kh, int kw, int sh, int sw, int ph, int pw, int dh, int dw, float *out,
            Act act);

// nn.Conv1d over (b, ic, len) after F.pad(x, (0, len_padded - len)) (the time
// encoder's right pad to a multiple of the stride, host.rs:633-640); weight
// (oc, ic, k) in GEMM order with kh = 1, kw = k.
void conv1d_right_padded(hipStream_t s, const float *x, int b, int ic, int len, int len_padded, const float *weight,
                         const float *bias, int oc, int k, int stride, int pad, float *out, Act act);

// Conv2d (any kernel, stride 1, weight in GEMM order) whose 2*C output
// channels feed F.glu(dim=1):
// out (b, C, oh, ow) = (y[c] + b[c]) * sigmoid(y[C+c] + b[C+c]). When `emb` is
// given, out[b][c][f][t] += emb_scale * emb[f][c] (the frequency embedding).
void conv2d_glu(hipStream_t s, const float *x, const float *skip, int b, int ic, int h, int w, const float *weight,
                const float *bias, int C, int kh, int kw, int ph, int pw, float *out, const float *emb,
                float emb_scale);

// nn.ConvTranspose along one axis (kernel k, stride st, no padding), cropped:
// x (b, ic, A, P) -> out (b, oc, a_out, P) with out[a'] = full[a' + crop].
// weight_packed is (st, oc, ic * taps) from pack_conv_transpose().
void conv_transpose_axis(hipStream_t s, const float *x, int b, int ic, int A, int P, const float *weight_packed,
                         const float *bias, int oc, int k, int st, int crop, int a_out, float *out, Act act);
int conv_transpose_taps(int k, int st);
// (ic, oc, k) checkpoint layout -> (st, oc, ic*taps) phase-major layout (host arrays).
void pack_conv_transpose(const float *w, int ic, int oc, int k, int st, float *packed);

// The frequency decoder's rewrite, conv2d 3x3 / padding 1 of (x + skip) from
// ic to 2C channels, bias, GLU (host.rs:682-759), by Winograd F(m x m, 3x3)
// (winograd.hip). winograd_tile() is the m a layer's widths take (0: the
// direct path; it decides which weights to prepare at load), winograd_applies()
// whether a call takes it (also fp32 MFMA precision). U is winograd_weights()
// of the PyTorch (2C, ic, 3, 3) weight, winograd_weight_floats() floats
// ((m+2)^2, 2C, ic); scratch holds winograd_scratch_floats(). skip may be null.
int winograd_tile(int ic, int C);
bool winograd_applies(int ic, int C, int F, int T);
int64_t winograd_weight_floats(int ic, int C);
int64_t winograd_scratch_floats(int B, int ic, int C, int F, int T);
void winograd_weights(const float *w, int oc, int ic, float *U);
void conv3x3_glu_winograd(hipStream_t s, const float *x, const float *skip, int B, int ic, int C, int F, int T,
                          const float *U, const float *bias, float *out, float *scratch);

// One DConv residual layer (crates/demucs-core/src/demucs/host.rs:985-1059), in
// place on x, whose rows are (b, f) of a (B, C, F, T) tensor (F = 1 for the
// waveform branch): conv1d k3 dilation `dil` -> GN(1) -> GELU -> 1x1 -> GN(1)
// -> GLU -> LayerScale -> +residual. `hbuf` holds dconv_hidden_floats()
// floats, `stats` 4*B*F doubles (both scratch). w1 is the PyTorch (H, C, 3)
// weight, w1_gemm the same in GEMM order (conv_gemm_weights with kh = 1,
// kw = 3), w1_t (may be null) the (C*3, H) transpose the narrow path reads
// (dconv_w1_transposed; made on the device when null).
// `gram` (dconv_gram_doubles(H) doubles from dconv_gram_weights, or null)
// lets the MFMA path take conv2's GroupNorm moments from the Gram matrix of
// its input instead of from a pass that computes conv2 for them.
void dconv_layer(hipStream_t s, float *x, int B, int C, int F, int T, int dil, const float *w1,
                 const float *w1_gemm, const float *w1_t, const float *b1, int H, const float *n1w,
                 const float *n1b, const float *w2, const float *b2, const float *n2w, const float *n2b,
                 const float *gamma, const double *gram, float *hbuf, double *stats);
int64_t dconv_gram_doubles(int H);
// W2^T W2, W2^T b2, sum_o W2[o], sum b2, sum b2^2 of conv2 (w2 (2C, H), b2 (2C)).
void dconv_gram_weights(hipStream_t s, const float *w2, const float *b2, int C, int H, double *out);
void dconv_w1_transposed(const float *w1, int C, int H, float *w1_t);

// The same layer with direct VALU kernels for hidden widths where MFMA tiles
// would be mostly padding (dconv.hip); returns false when it does not apply.
// Floats of the hidden-activation scratch `hbuf` that dconv_layer needs.
int64_t dconv_hidden_floats(int rows, int H, int T);
bool dconv_narrow_applies(int C, int H);
// Both layers of a depth-2 DConv (`dconv_forward`, host.rs:984-1059; dilations
// 1 and 2) in one launch, one workgroup per (b, f) row held in LDS; returns
// false (nothing launched) unless C = 48 or 96 with H = C/8 and T <= 384.
// w1_t is each layer's w1 as (C*3, H) (dconv_w1_transposed).
struct DConvRowLayer {
    const float *w1_t, *b1, *n1w, *n1b, *w2, *b2, *n2w, *n2b, *gamma;
};
bool dconv_rows(hipStream_t s, float *x, int B, int C, int F, int T, int H, const DConvRowLayer layers[2]);
bool dconv_layer_narrow(hipStream_t s, float *x, int B, int C, int F, int T, int dil, const float *w1,
                        const float *w1_t, const float *b1, int H, const float *n1w, const float *n1b,
                        const float *w2, const float *b2, const float *n2w, const float *n2b, const float *gamma,
                        float *hbuf);

// out (z, M, N) = W (M, K) . x (z, K, N) + bias[m]  (1x1 conv / channel mixer).
void pointwise(hipStream_t s, const float *w, const float *bias, const float *x, int batches, int M, int K, int N,
               float *out, Act act);

// Linear on token rows: out[z][m][n] = x[z][m][:] . W[n][:] + bias[n], with the
// requested tail. x rows have stride ldx, out rows stride ldo.
enum LinearTail { TAIL_BIAS = 0, TAIL_BIAS_GELU = 1, TAIL_RESIDUAL_SCALE = 2 };
void linear(hipStream_t s, const float *x, int64_t ldx, int64_t x_batch_stride, const float *w, const float *bias,
            int batches, int M, int K, int N, float *out, int64_t ldo, int64_t out_batch_stride, LinearTail tail,
            const float *residual, const float *gamma, double *stats);

// An fp32 operand stored as `count` bf16 planes (x = x_0 + ... + x_{count-1},
// each plane round-to-nearest-even of what the previous ones leave): plane q
// of element i is p[q * stride + i]. count = 3 holds every fp32 value
// exactly; count = 1 is plain bf16.
struct Planes {
    unsigned short *p = nullptr;
    int64_t stride = 0;
    int count = 0;
    Planes offset(int64_t elements) const { return Planes{p ? p + elements : nullptr, stride, count}; }
};
// K and V of one attention problem as the three-plane kernel reads them:
// K planes [plane][b][token][ldk] (head h at column 64 h); V^T planes
// [plane][(b * heads + h) * 64 + d][ldvt], tokens of every 16-token group
// stored in the order 0-3, 8-11, 4-7, 12-15 (vt_token_pos: bits 2 and 3
// swapped), zeros from n_k up to ldvt, a multiple of 32.
struct KVPlanes {
    unsigned short *k = nullptr, *vt = nullptr;
    int64_t k_stride = 0, k_bs = 0, ldk = 0;  // plane, batch and row strides (bf16 elements)
    int64_t vt_stride = 0, ldvt = 0;          // plane and row strides
};
__host__ __device__ inline int64_t vt_token_pos(int64_t t) { return (t & ~int64_t(12)) | ((t & 4) << 1) | ((t & 8) >> 1); }
inline int64_t kv_ldvt(int64_t n_k) { return (n_k + 31) / 32 * 32; }
// x (n floats) -> planes.
void split_to_planes(hipStream_t s, const float *x, int64_t n, Planes out);
// linear() over plane operands on the bf16 matrix cores (gemm_planes.h):
// x rows at z * x_batch_stride + m * ldx of every plane, W (N, K) row-major
// planes. The result goes to `out` (fp32), or, when out_planes.p is set, to
// out_planes (same indexing; the bias + GELU tail only) and `out` is unused. Plane products (i, j) with
// i + j < count are summed, so count = 3 is an fp32-accurate product.
void linear_planes(hipStream_t s, Planes x, int64_t ldx, int64_t x_batch_stride, Planes w, const float *bias,
                   int batches, int M, int K, int N, float *out, Planes out_planes, int64_t ldo,
                   int64_t out_batch_stride, LinearTail tail, const float *residual, const float *gamma,
                   double *stats);

// The attention in-projection on planes for the three-plane attention: the
// N = q_cols + 2 D output columns of token m of batch z (plus bias) go to q
// (fp32, z * M * D + m * D) for the first q_cols (0 or D), then to the K and
// V^T planes of `kv` (KVPlanes layout, V^T rows of kv.ldvt >= M rounded up
// to 32, whose padding the caller zeroes when M is not a multiple of 32).
void linear_qkv_planes(hipStream_t s, Planes x, int64_t ldx, int64_t x_batch_stride, Planes w, const float *bias,
                       int batches, int M, int K, int N, int q_cols, float *q, const KVPlanes &kv);

// Channel mixer reading transformer tokens: out (b, M, F*T) with
// out[z][m][f*T + t] = W[m] . tok[z][t*F + f] + bias[m] (F = 1: token = t).
void tokens_to_channels(hipStream_t s, const float *tok, int b, int F, int T, int D, const float *w, const float *bias,
                        int M, float *out);

// ---------------- attention (attention.hip) ----------------
// Fused softmax(q k^T * scale) v per (batch, head); q/k/v/out are token-major
// with the head's 64 lanes at column h*64 of rows of stride ld*.
void attention(hipStream_t s, const float *q, int64_t ldq, const float *k, int64_t ldk, const float *v, int64_t ldv,
               float *out, int64_t ldo, int batch, int heads, int n_q, int n_k, int d_head, float scale,
               int64_t q_batch_stride, int64_t kv_batch_stride, int64_t out_batch_stride);
// Up to two independent problems (same scale) in one launch, e.g. the two
// branches of a transformer layer; each as the arguments of attention().
// fp32 K / V rows (b * kv_bs + token * ld + 64 h + d) -> KVPlanes.
void kv_to_planes(hipStream_t s, const float *k, int64_t ldk, const float *v, int64_t ldv, int64_t kv_bs, int batch,
                  int heads, int n_k, const KVPlanes &out);
// Whether the fp32 precision's attention runs on the three-plane kernel
// (DMX_ATT_PLANES=0 keeps the fp32-MFMA kernel).
bool attention_planes_enabled();

struct AttentionArgs {
    const float *q;
    int64_t ldq;
    const float *k;
    int64_t ldk;
    const float *v;
    int64_t ldv;
    float *out;
    int64_t ldo;
    int batch, heads, n_q, n_k, d_head;
    int64_t q_batch_stride, kv_batch_stride, out_batch_stride;
    // When set, the output goes to these bf16 planes (same indexing as out),
    // and out is unused.
    Planes out_planes{};
    // When set, K and V come from these planes (the three-plane kernel; k, v,
    // ldk, ldv and kv_batch_stride are unused).
    KVPlanes kv{};
};
void attention_grouped(hipStream_t s, const AttentionArgs *probs, int count, float scale);

// ---------------- norms / elementwise (norm.hip) ----------------
void layer_norm_rows(hipStream_t s, const float *x, int rows, int dim, const float *w, const float *b, float *out,
                     const float *add, int add_rows);
// The same (dim = 512, no add) with the output written as bf16 planes.
void layer_norm_planes(hipStream_t s, const float *x, int rows, int dim, const float *w, const float *b, Planes out);
// (b, c, positions) channel-major -> token rows (b, T*F, c) reordered token = t*F + f,
// LayerNorm over c, then + pos[token] (pos may be null).
void channels_to_tokens_ln(hipStream_t s, const float *x, int b, int c, int F, int T, const float *w,
                           const float *bias, const float *pos, float pos_weight, float *out);
// GroupNorm(1, C) over whole (L, C) token planes from f64 stats (2 per batch), in place.
void group_norm_tokens_apply(hipStream_t s, float *x, int b, int L, int C, const double *stats, const float *w,
                             const float *bias);
// nn.GroupNorm(groups, c) over (b, c, inner).
void group_norm(hipStream_t s, const float *x, int b, int c, int inner, int groups, const float *w, const float *bias,
                float *out, double *stats_scratch);
void glu(hipStream_t s, const float *x, int b, int c2, int inner, float *out);
void gelu(hipStream_t s, const float *x, int64_t n, float *out);
void zero_doubles(hipStream_t s, double *p, int64_t n);
void zero_floats(hipStream_t s, float *p, int64_t n);
// dst[r][t] = t < n_copy ? src[r * src_ld + t] : 0 for t < dst_len.
void copy_rows(hipStream_t s, const float *src, int64_t rows, int64_t src_ld, int64_t n_copy, float *dst,
               int64_t dst_len);

// ---------------- spectral / framing (spectral.hip) ----------------
// _spec + pack (CaC) + per-batch normalisation of both branches:
// mix (b, 2, L) -> xspec (b, 4, nfft/2, le) normalised, xwave (b, 2, L) normalised,
// norms[4*b] = (mean, std, mean_t, std_t) per batch (f32).
void spec_and_normalise(hipStream_t s, const float *mix, int b, int L, int nfft, float *spec_raw_frames,
                        float *xspec, float *xwave, float *norms, double *stats, const float *twiddles);
// CaC output (b, 4S, nfft/2, le) + time branch (b, 2S, L) -> stems (b, S, 2, L)
// with both denormalisations and the iSTFT.
void ispec_and_sum(hipStream_t s, const float *xspec, const float *xtime, int b, int S, int L, int nfft, int le,
                   const float *norms, float *frames_scratch, float *stems, const float *twiddles);
// Raw STFT pieces for op-level checks.
void stft_cac_raw(hipStream_t s, const float *mix, int b, int L, int nfft, float *frames_out, float *xspec_out,
                  const float *twiddles);
void make_twiddles(int nfft, float *host_out);  // nfft/2 complex (cos, -sin) pairs

// ---------------- chunking / overlap-add (pipeline.hip) ----------------
void mix_moments(hipStream_t s, const float *mix, int64_t samples, double *stats);
void build_chunks(hipStream_t s, const float *mix, int64_t mix_len, const double *stats, int group, const int64_t *starts,
                  const int64_t *lengths, int64_t seg, int64_t view_len, int64_t shift_offset, int64_t max_shift,
                  float *out);
void ola_accumulate(hipStream_t s, const float *chunk_out, int group, const int64_t *starts, const int64_t *lengths,
                    int64_t seg, int rows, int64_t view_len, const float *weight, float *acc, float *sum_w);
// Finishes output samples [lo, hi) of every row from the pass's sums (modes in pipeline.hip).
void ola_finish(hipStream_t s, const float *acc, const float *sum_w, int rows, int64_t view_len, int64_t trim,
                int64_t lo, int64_t hi, int64_t samples, const double *stats, float scale, int mode, float *stems,
                const uint8_t *row_mask);
void bag_accumulate(hipStream_t s, const float *net_out, int64_t group_batch, int sources, int64_t per_source,
                    const float *weights, float *combined, int first);
void bag_divide(hipStream_t s, float *combined, int64_t group_batch, int sources, int64_t per_source,
                const float *totals);

}  // namespace dmx
