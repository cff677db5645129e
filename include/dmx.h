/*
 * dmx.h — C-ABI of the MI355X-native HTDemucs v4 inference backend.
 *
 * This is the drop-in boundary for the reference's segment forward. A new
 * `Backend::Hip` variant in the reference facade binds these functions over
 * FFI; everything above them (Demucs::load / separate / separate_with_progress /
 * StemSelection) keeps its contract. Plain pointers and sizes only.
 *
 * Conventions
 *  - Every function returning `int` returns DMX_OK (0) on success, otherwise a
 *    DMX_ERR_* code, and leaves a message in the calling thread's
 *    dmx_last_error(). Codes mirror the variants of the reference's
 *    `Error` enum the path can raise (crates/demucs-core/src/error.rs:4-55).
 *  - Host tensors are row-major f32 in PyTorch layout.
 *  - One runner is used by one thread at a time; distinct runners are
 *    independent. All device work of a runner goes to its own HIP stream.
 */
#ifndef DMX_H
#define DMX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum dmx_status {
    DMX_OK = 0,
    DMX_ERR_SHAPE = 1,          /* Error::Shape */
    DMX_ERR_CONFIG = 2,         /* Error::Config */
    DMX_ERR_MISSING_WEIGHT = 3, /* Error::MissingWeight */
    DMX_ERR_WEIGHT_SHAPE = 4,   /* Error::WeightShape */
    DMX_ERR_UNSUPPORTED = 5,    /* Error::UnsupportedModel */
    DMX_ERR_GPU = 6,            /* Error::Gpu */
    DMX_ERR_MEMORY = 7,         /* Error::Memory */
    DMX_ERR_ARGUMENT = 8,       /* null pointer / bad enum at the C boundary */
    DMX_ERR_CHECKPOINT = 9,     /* Error::Checkpoint / Error::Pickle (dmx_ckpt.h) */
    DMX_ERR_IO = 10,            /* Error::Io (dmx_ckpt.h, dmx_audio.h) */
    DMX_ERR_AUDIO = 11          /* Error::Audio (dmx_audio.h) */
};

enum dmx_precision {
    /* fp32 results (parity: per-stem SNR >= 60 dB, activations within 1e-3):
     * convolutions and attention on the fp32 matrix cores; the transformer
     * linears on the bf16 matrix cores over three bf16 planes per operand
     * (x = x0 + x1 + x2, all 24 significant bits), an fp32-accurate product. */
    DMX_PRECISION_FP32 = 0,
    /* bf16 MFMA inputs for attention/GEMMs, fp32 softmax/norms/output (>= 40 dB) */
    DMX_PRECISION_BF16 = 1,
    /* fp32 MFMA for every contraction, the linears included (same parity bar
     * as DMX_PRECISION_FP32) */
    DMX_PRECISION_FP32_MFMA = 2
};

/* One named weight tensor, keyed by its checkpoint name
 * (e.g. "encoder.0.conv.weight", "crosstransformer.layers.1.cross_attn.in_proj_weight").
 * Key set and shapes: crates/demucs-core/src/demucs/weights.rs:224-578. */
typedef struct dmx_tensor {
    const char *name;
    const float *data;
    int32_t ndim;
    int64_t shape[4];
} dmx_tensor;

/* HtdemucsConfig (crates/demucs-core/src/demucs/config.rs:18-71). */
typedef struct dmx_config {
    int32_t sources;         /* 4 */
    int32_t audio_channels;  /* 2 */
    int32_t samplerate;      /* 44100 */
    double segment;          /* seconds; training_length = int(segment * samplerate) */
    int32_t channels;        /* 48 */
    int32_t growth;          /* 2 */
    int32_t nfft;            /* 4096 */
    int32_t depth;           /* 4 */
    int32_t stride;          /* 4 */
    int32_t kernel_size;     /* 8 */
    int32_t context;         /* 1 */
    double freq_emb;         /* 0.2 */
    double emb_scale;        /* 10 */
    int32_t cac;             /* 1 */
    int32_t bottom_channels; /* 512 */
    int32_t t_layers;        /* 5 */
    int32_t t_heads;         /* 8 */
    double t_hidden_scale;   /* 4.0 */
    double t_max_period;     /* 10000 */
    double t_weight_pos_embed; /* 1.0 */
} dmx_config;

/* HtdemucsConfig::default (config.rs:43-71). */
void dmx_config_default(dmx_config *cfg);
/* HtdemucsConfig::training_length (config.rs:222-224). */
int64_t dmx_config_training_length(const dmx_config *cfg);

/* Message for the last failing call on this thread ("" if none). */
const char *dmx_last_error(void);

/* Number of visible HIP devices (0 when none; never fails). */
int dmx_device_count(void);

typedef struct dmx_runner dmx_runner;
typedef struct dmx_pending dmx_pending;

/* Builds a runner: validates the config (HtdemucsConfig::validate, config.rs:239-273),
 * checks every weight's shape, uploads the weights once.
 * Replaces GpuHtdemucsRunner::with_selector (crates/demucs-core/src/gpu/htdemucs.rs:2377-2400)
 * as called from make_runner (crates/demucs-core/src/api.rs:1014-1036). */
int dmx_runner_create(const dmx_tensor *weights, size_t n_weights, const dmx_config *cfg,
                      int device_ordinal, int precision, dmx_runner **out);
void dmx_runner_destroy(dmx_runner *runner);
/* "hip:<device name>" (describe / backend_tag, api.rs:1038-1045, 821). */
const char *dmx_runner_backend_tag(const dmx_runner *runner);
/* The runner's main hipStream_t, for callers that order their own device work
 * after it: the device entry points finish their work on it (a group queued by
 * dmx_forward_start may run on the runner's second stream pair; dmx_synchronize
 * waits for every stream). */
void *dmx_runner_stream(dmx_runner *runner);
int dmx_synchronize(dmx_runner *runner);

/* SegmentForward::start (crates/demucs-core/src/demucs/pipeline.rs:178-190):
 * queues a forward of `mix` (batch, channels, length), length <= training_length,
 * and returns with the work in flight. The host array may be reused on return.
 * Groups in flight are not limited (the caller of the reference keeps two);
 * each holds a pinned staging slot of the runner until it is collected, and
 * consecutive groups run on alternating stream pairs so they overlap. Slots
 * are reused, so steady state allocates nothing. */
int dmx_forward_start(dmx_runner *runner, const float *mix, int64_t batch, int64_t channels,
                      int64_t length, dmx_pending **out);
/* SegmentForward::collect: waits for that group only and writes
 * (batch, sources, channels, length) into `stems`; frees `pending`.
 * A null argument or a group of another runner is an error that leaves the
 * group pending; groups may be collected in any order. */
int dmx_forward_collect(dmx_runner *runner, dmx_pending *pending, float *stems);
/* Htdemucs::forward (crates/demucs-core/src/demucs/host.rs:202-520), synchronous. */
int dmx_forward(dmx_runner *runner, const float *mix, int64_t batch, int64_t channels,
                int64_t length, float *stems);
/* Same forward with device-resident input and output (no host copies),
 * enqueued on the runner's stream. */
int dmx_forward_device(dmx_runner *runner, const float *d_mix, int64_t batch, int64_t channels,
                       int64_t length, float *d_stems);

/* The cross-transformer stack alone, device-resident
 * (Htdemucs::transformer_forward, host.rs:830-946): d_spec is (batch, C, freqs, frames),
 * d_time is (batch, C, time_len), C = bottom_channels; outputs have the same shapes. */
int dmx_crosstransformer_device(dmx_runner *runner, const float *d_spec, const float *d_time,
                                int64_t batch, int64_t freqs, int64_t frames, int64_t time_len,
                                float *d_spec_out, float *d_time_out);

/* TraceSink (host.rs:117-125): `wants(name)` is asked before a named activation
 * is copied back; `record` receives it in the reference's layout. */
typedef int (*dmx_trace_wants_fn)(const char *name, void *user);
typedef void (*dmx_trace_record_fn)(const char *name, const int64_t *shape, int32_t ndim,
                                    const float *data, void *user);
int dmx_set_trace(dmx_runner *runner, dmx_trace_wants_fn wants, dmx_trace_record_fn record,
                  void *user);

/* SeparateOptions (pipeline.rs:16-38) plus the group size DEMUCS_BATCH
 * (pipeline.rs:491-502). segment <= 0 means the model's segment. */
typedef struct dmx_separate_options {
    int32_t shifts;
    double overlap;
    double transition_power;
    double segment;
    int32_t batch_chunks;
} dmx_separate_options;
void dmx_separate_options_default(dmx_separate_options *opts);

typedef void (*dmx_progress_fn)(size_t done, size_t total, void *user);

/* Demucs::separate_with_options (api.rs:438-451) for one network or a bag:
 * global normalisation (streaming.rs:52-85), chunking + triangular overlap-add
 * (streaming.rs:296-400), the shift trick (pipeline.rs:380-515), the bag's
 * weighted combine (api.rs:319-371) and StemSelection (api.rs:170-178, 559-605).
 *  nets[n_nets], bag_weights (n_nets x sources, row-major; NULL = identity-free
 *  single network), stems_wanted[sources] (NULL = all).
 *  left/right: host samples; stems_out: (sources, 2, samples) host, rows of
 *  unwanted stems are left untouched.
 * The mix goes up through the runner's pinned staging; each chunk group's
 * finished output samples are read back while later groups compute, the
 * reference's OlaRing flush after each segment (streaming.rs:96-261,
 * :389-394). `progress(done, total, user)` runs on the calling thread after
 * each group; it does not change the schedule on the GPU. */
int dmx_separate(dmx_runner *const *nets, const float *bag_weights, int32_t n_nets,
                 const uint8_t *stems_wanted, const float *left, const float *right,
                 int64_t samples, int32_t sample_rate, const dmx_separate_options *opts,
                 dmx_progress_fn progress, void *user, float *stems_out);

/* The stems of output samples [start, start + frames), handed over in
 * order: rows[2 * s + c] points at `frames` samples of stem s, channel c
 * (NULL for a stem not wanted). The memory is the runner's and is valid
 * only during the call. Return 0 to go on; anything else stops the
 * separation, which then returns DMX_ERR_IO. */
typedef int (*dmx_emit_fn)(int64_t start, int64_t frames, const float *const *rows, void *user);
/* Separate::separate_emit / separate_streaming_normalized_mix
 * (crates/demucs-core/src/api.rs:265-298, :697-785): dmx_separate, but
 * instead of filling a (sources, 2, samples) host array it hands each
 * finished region to `emit` on the calling thread as soon as its readback
 * has landed (the reference's on_frame, a region at a time), while later
 * chunk groups still compute. Denormalised, like dmx_separate's stems. */
int dmx_separate_emit(dmx_runner *const *nets, const float *bag_weights, int32_t n_nets,
                      const uint8_t *stems_wanted, const float *left, const float *right,
                      int64_t samples, int32_t sample_rate, const dmx_separate_options *opts,
                      dmx_progress_fn progress, void *user, dmx_emit_fn emit, void *emit_user);
/* Same with device-resident mix (2, samples) and stems (sources, 2, samples),
 * enqueued on the runner's stream; without a progress callback it returns
 * before the GPU has finished. */
int dmx_separate_device(dmx_runner *const *nets, const float *bag_weights, int32_t n_nets,
                        const uint8_t *stems_wanted, const float *d_mix, int64_t samples,
                        int32_t sample_rate, const dmx_separate_options *opts,
                        dmx_progress_fn progress, void *user, float *d_stems);

#ifdef __cplusplus
}
#endif

#endif /* DMX_H */
