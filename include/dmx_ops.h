/*
 * dmx_ops.h — per-kernel entry points of the HIP backend, for parity tests and
 * micro-benchmarks. Each mirrors one dispatch wrapper of the reference's
 * device `Kernels` (crates/demucs-core/src/gpu/kernels.rs), which the
 * reference's own GPU tests drive one kernel at a time (core/tests/gpu_*.rs).
 *
 * All tensor pointers are DEVICE pointers; work is enqueued on `stream`
 * (a hipStream_t, NULL = the default stream) and not synchronised.
 * Return DMX_OK or a DMX_ERR_* code with dmx_last_error() set.
 */
#ifndef DMX_OPS_H
#define DMX_OPS_H

#include <stdint.h>

#include "dmx.h"

#ifdef __cplusplus
extern "C" {
#endif

enum { DMX_ACT_NONE = 0, DMX_ACT_GELU = 1 };

/* MFMA input precision (a dmx_precision value) of the contractions this
 * thread enqueues through the dmx_op_* entry points below (linear, conv2d,
 * conv2d_glu, conv_transpose, dconv_layer, pointwise, attention);
 * accumulation and every output stay fp32. Per thread, default
 * DMX_PRECISION_FP32 (dmx_op_linear then splits x and the weight into three
 * bf16 planes each before the product). The bf16 variant of a runner is chosen at dmx_runner_create instead.
 * No counterpart in the reference, whose device path is fp32 only; it exists
 * so the bf16 kernels can be tested one at a time like the fp32 ones. */
int dmx_op_set_precision(int precision);
enum { DMX_TAIL_BIAS = 0, DMX_TAIL_BIAS_GELU = 1, DMX_TAIL_RESIDUAL_SCALE = 2 };

/* conv2d_gemm_into (kernels.rs:3089-3257) as an implicit GEMM: x (b, ic, h, w),
 * weight (oc, ic, kh, kw), optional skip added to x while gathering. */
int dmx_op_conv2d(void *stream, const float *x, const float *skip, int b, int ic, int h, int w, const float *weight,
                  const float *bias, int oc, int kh, int kw, int sh, int sw, int ph, int pw, int dh, int dw, int act,
                  float *out);
/* conv + F.glu(dim=1) fused (stride 1): out (b, C, oh, ow); emb (F, C) optional. */
int dmx_op_conv2d_glu(void *stream, const float *x, const float *skip, int b, int ic, int h, int w,
                      const float *weight, const float *bias, int C, int kh, int kw, int ph, int pw,
                      const float *emb, float emb_scale, float *out);
/* conv_transpose2d_into (kernels.rs:4011-4151) along one axis, cropped: x (b, ic, A, P),
 * weight (ic, oc, k) -> out (b, oc, a_out, P) = full[crop : crop + a_out]. */
int dmx_op_conv_transpose(void *stream, const float *x, int b, int ic, int A, int P, const float *weight,
                          const float *bias, int oc, int k, int st, int crop, int a_out, int act, float *out);
/* One DConv residual layer in place on x (B, C, F, T) whose rows are (b, f). */
int dmx_op_dconv_layer(void *stream, float *x, int B, int C, int F, int T, int dilation, const float *w1,
                       const float *b1, int hidden, const float *n1w, const float *n1b, const float *w2,
                       const float *b2, const float *n2w, const float *n2b, const float *gamma);
/* dconv_forward (crates/demucs-core/src/demucs/host.rs:984-1059): both layers of a
 * depth-2 DConv (dilations 1 and 2) in place on x (B, C, F, T) whose rows are (b, f).
 * params holds 18 device pointers, 9 per layer in the order
 * w1 (H, C, 3), b1, norm1 weight, norm1 bias, w2 (2C, H, 1), b2, norm2 weight,
 * norm2 bias, LayerScale; H = hidden. Rows of at most 384 positions with
 * C = 48 or 96 run as one launch with the row in LDS. */
int dmx_op_dconv(void *stream, float *x, int B, int C, int F, int T, int hidden, const float *const *params);
/* gemm_into_epilogue (kernels.rs:1531-1621): out (rows, N) = x (rows, K) . W^T + bias
 * with the tail: GELU, or residual + gamma * (.) */
int dmx_op_linear(void *stream, const float *x, int rows, int K, const float *w, const float *bias, int N, int tail,
                  const float *residual, const float *gamma, float *out);
/* out (z, M, N) = W (M, K) . x (z, K, N) + bias[m] */
int dmx_op_pointwise(void *stream, const float *w, const float *bias, const float *x, int batches, int M, int K,
                     int N, float *out);
/* attention_stage (htdemucs.rs:1416-1513) fused: q (B, n_q, H*64), k/v (B, n_k, H*64) -> out (B, n_q, H*64). */
int dmx_op_attention(void *stream, const float *q, const float *k, const float *v, float *out, int batch, int heads,
                     int n_q, int n_k, float scale);
/* Two attention problems of the same batch, heads and scale in one launch, as
 * the runner issues the two branches of each transformer layer (spectral and
 * waveform tokens). No counterpart in the reference, which dispatches each
 * branch's attention on its own; it is the launch bench.py's roofline times. */
int dmx_op_attention_pair(void *stream, const float *q0, const float *k0, const float *v0, float *out0, int n_q0,
                          int n_k0, const float *q1, const float *k1, const float *v1, float *out1, int n_q1,
                          int n_k1, int batch, int heads, float scale);
/* The three-plane attention's operands, for timing its kernel alone (no
 * counterpart in the reference): dmx_op_kv_planes writes K and V of one
 * problem (batch, n_k, heads * 64 floats each) as three bf16 planes, K into
 * k_planes (3 * batch * n_k * heads * 64 elements) and V transposed per head
 * into vt_planes (3 * batch * heads * 64 * ldvt elements, ldvt = n_k rounded
 * up to a multiple of 32); dmx_op_attention_pair_planes is
 * dmx_op_attention_pair over such planes, one kernel launch. Both enqueue
 * only (no synchronisation). */
int dmx_op_kv_planes(void *stream, const float *k, const float *v, int batch, int heads, int n_k,
                     unsigned short *k_planes, unsigned short *vt_planes);
int dmx_op_attention_pair_planes(void *stream, const float *q0, unsigned short *kp0, unsigned short *vtp0,
                                 float *out0, int n_q0, int n_k0, const float *q1, unsigned short *kp1,
                                 unsigned short *vtp1, float *out1, int n_q1, int n_k1, int batch, int heads,
                                 float scale);
int dmx_op_layer_norm(void *stream, const float *x, int rows, int dim, const float *w, const float *b, float *out);
int dmx_op_group_norm(void *stream, const float *x, int b, int c, int inner, int groups, const float *w,
                      const float *bias, float *out);
int dmx_op_glu(void *stream, const float *x, int b, int c2, int inner, float *out);
int dmx_op_gelu(void *stream, const float *x, int64_t n, float *out);
/* stft_cac_into + batch_moments + batch_normalize (kernels.rs:3662-3870):
 * mix (b, 2, L) -> xspec (b, 4, 2048, le), xwave (b, 2, L), norms (b, 4) = (mean, std, mean_t, std_t). */
int dmx_op_spec_normalise(void *stream, const float *mix, int b, int L, float *xspec, float *xwave, float *norms);
/* dmx_op_spec_normalise without allocating: no counterpart in the reference.
 * For callers that cannot call hipMalloc (code under HIP graph capture,
 * serving loops, harnesses that forbid it). The STFT frames and moments live
 * in the library's fixed device scratch (about 22 MB per GPU, held until the
 * process ends): at most 64 batch rows and b * ceil(L / 1024) <= 672 (two
 * 7.8 s segments); larger inputs are a DMX_ERR_SHAPE error. Asynchronous on
 * `stream`. The first call on a device sets the scratch up (a synchronous
 * 32 KB table copy): make it before capturing. Calls on one GPU share its
 * scratch, so calls that overlap on one GPU race. */
int dmx_op_spec_normalise_noalloc(void *stream, const float *mix, int b, int L, float *xspec, float *xwave,
                                  float *norms);
/* ispec_cac_into + final sum (kernels.rs:3877-3973): xspec (b, 16, 2048, le), xtime (b, 8, L),
 * norms (b, 4) -> stems (b, 4, 2, L). */
int dmx_op_ispec_sum(void *stream, const float *xspec, const float *xtime, int b, int L, const float *norms,
                     float *stems);

#ifdef __cplusplus
}
#endif

#endif /* DMX_OPS_H */
