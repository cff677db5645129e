/*
 * oracle.h — CPU restatement of the reference's HTDemucs host backend.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity checker and the timed
 * CPU baseline ("restated reference CPU backend"). Only tests/, the smoke test
 * and bench.py's cpu_baseline leg may load it; the product library never links,
 * loads or calls it.
 *
 * Each function restates a function of eclipse005/demucs-wgpu's Rust CPU path
 * (crates/demucs-core/src/...), cited at its definition in oracle.cpp. The
 * reference itself is Rust (cargo is absent here), so it cannot be built;
 * this restatement is pinned by the reference's own known-answer tests and by
 * independent float64 torch.nn.functional / torch.stft computations (tests/).
 */
#ifndef DMX_ORACLE_H
#define DMX_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#include "../include/dmx.h"

#ifdef __cplusplus
extern "C" {
#endif

const char *oracle_last_error(void);
void oracle_set_threads(int threads);
int oracle_get_threads(void);

/* ---- single operators (layouts as in PyTorch, row-major) ---- */
void oracle_sgemm(int64_t m, int64_t n, int64_t k, const float *a, int64_t a_rs, int64_t a_cs,
                  const float *b, int64_t b_rs, int64_t b_cs, float *c, int64_t ldc);
int oracle_conv2d(const float *x, int64_t batch, int64_t ic, int64_t h, int64_t w,
                  const float *weight, const float *bias, int64_t oc, int64_t kh, int64_t kw,
                  int64_t sh, int64_t sw, int64_t ph, int64_t pw, int64_t dh, int64_t dw,
                  float *out);
int oracle_conv_transpose2d(const float *x, int64_t batch, int64_t ic, int64_t h, int64_t w,
                            const float *weight, const float *bias, int64_t oc, int64_t kh,
                            int64_t kw, int64_t sh, int64_t sw, float *out);
int oracle_group_norm(const float *x, int64_t batch, int64_t channels, int64_t inner,
                      int64_t groups, const float *weight, const float *bias, float *out);
int oracle_group_norm_glu(const float *x, int64_t batch, int64_t channels, int64_t inner,
                          int64_t groups, const float *weight, const float *bias, float *out);
int oracle_layer_norm_rows(const float *x, int64_t rows, int64_t dim, const float *weight,
                           const float *bias, float *out);
int oracle_glu(const float *x, int64_t batch, int64_t channels, int64_t inner, float *out);
void oracle_gelu(const float *x, int64_t n, float *out);
float oracle_gelu_scalar(float x);
float oracle_mean(const float *x, int64_t n);
float oracle_std_unbiased(const float *x, int64_t n);
int oracle_attention_head(const float *q, const float *k, const float *v, int64_t n_q,
                          int64_t n_k, int64_t d_head, float scale, float *out);
/* nn.MultiheadAttention on (batch, n, dim) with split q/k/v weights (dim, dim). */
int oracle_multi_head_attention(const float *query, const float *key, int64_t batch,
                                int64_t n_q, int64_t n_k, int64_t dim, int64_t heads,
                                const float *wq, const float *bq, const float *wk,
                                const float *bk, const float *wv, const float *bv,
                                const float *wo, const float *bo, float *out);
int oracle_dconv(const float *x, int64_t rows, int64_t channels, int64_t t, const dmx_tensor *w,
                 size_t n, const char *prefix, float *out);
void oracle_hann_window(int64_t n, float *out);
void oracle_fft(const float *re, const float *im, int64_t n, int inverse, double *out_re,
                double *out_im);
/* torch.stft(center=True, reflect, periodic Hann, onesided): (batch, samples) ->
 * (batch, n_fft/2+1, frames) complex as separate re/im planes. */
int oracle_stft(const float *x, int64_t batch, int64_t samples, int64_t n_fft, int64_t hop,
                int normalized, float *out_re, float *out_im, int64_t *frames_out);
int oracle_istft(const float *re, const float *im, int64_t batch, int64_t bins, int64_t frames,
                 int64_t n_fft, int64_t hop, int normalized, int64_t length, float *out,
                 int64_t *out_len);
int oracle_pad1d_reflect(const float *x, int64_t length, int64_t left, int64_t right, float *out);
/* HTDemucs._spec + CaC packing: (b, c, L) -> (b, 2c, nfft/2, ceil(L/hop)). */
int oracle_spec_cac(const float *mix, int64_t batch, int64_t channels, int64_t length,
                    int64_t nfft, float *out);
/* _mask inverse packing + _ispec: (b, 4s... ) CaC (b, s*2*2, nfft/2, le) -> (b, s, 2, length). */
int oracle_ispec_cac(const float *x, int64_t batch, int64_t sources, int64_t bins, int64_t le,
                     int64_t nfft, int64_t length, float *out);
void oracle_positions_2d(int64_t dim, int64_t height, int64_t width, float max_period,
                         float *out);
void oracle_positions_1d(int64_t length, int64_t dim, float max_period, float *out);
void oracle_transition_weight(int64_t segment_length, double power, float *out);
/* ShiftRng(seed).randint(max) `count` times (pipeline.rs:136-151). */
void oracle_shift_rng(uint64_t seed, int64_t max, int64_t count, int64_t *out);
/* scan_norm (streaming.rs:52-78): mean and unbiased std (+1e-8) of the channel mean. */
void oracle_scan_norm(const float *wav, int64_t batch, int64_t channels, int64_t length,
                      float *mean, float *std);

/* ---- the model ---- */
typedef struct oracle_model oracle_model;
oracle_model *oracle_model_create(const dmx_tensor *weights, size_t n, const dmx_config *cfg);
void oracle_model_destroy(oracle_model *model);
int64_t oracle_model_training_length(const oracle_model *model);
int oracle_forward(oracle_model *model, const float *mix, int64_t batch, int64_t channels,
                   int64_t length, float *out, dmx_trace_wants_fn wants,
                   dmx_trace_record_fn record, void *user);
int oracle_transformer_forward(oracle_model *model, const float *x, const float *xt,
                               int64_t batch, int64_t freqs, int64_t frames, int64_t time_len,
                               float *x_out, float *xt_out, dmx_trace_wants_fn wants,
                               dmx_trace_record_fn record, void *user);

/* ---- chunking / overlap-add / shifts / bag (pipeline.rs, streaming.rs, api.rs) ----
 * `forward` (optional) replaces the model forward: it receives a padded group
 * (batch, channels, segment) and writes (batch, sources, channels, segment). */
typedef int (*oracle_forward_fn)(const float *padded, int64_t batch, int64_t channels,
                                 int64_t length, float *out, void *user);
int oracle_separate(oracle_model *const *nets, const float *bag_weights, int32_t n_nets,
                    const uint8_t *stems_wanted, const float *left, const float *right,
                    int64_t samples, int32_t sample_rate, const dmx_separate_options *opts,
                    oracle_forward_fn forward, void *forward_user, int32_t sources,
                    float *stems_out);
/* stream_split_pass on an already-normalised (batch, channels, length) mix,
 * without denormalisation, for the identity-forward OLA tests. */
int oracle_split_pass(const float *mix, int64_t batch, int64_t channels, int64_t length,
                      int64_t segment_length, double overlap, double transition_power,
                      int64_t shift_offset, int64_t max_shift, int32_t batch_chunks,
                      int32_t sources, oracle_forward_fn forward, void *user, float *out);

#ifdef __cplusplus
}
#endif

#endif
