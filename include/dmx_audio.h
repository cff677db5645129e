/*
 * dmx_audio.h — audio files and the stem comparison of the HIP backend's
 * command-line front end: RIFF/WAVE reading and writing, a streaming float
 * WAV writer, and the reference's element-wise comparison metric.
 *
 * Host-only code in libdmx.so (no GPU involved). Status codes and
 * dmx_last_error() as in dmx.h; audio format problems are DMX_ERR_AUDIO
 * (the reference's Error::Audio), file system problems DMX_ERR_IO.
 * Sample buffers are channel-major: channel c occupies
 * data[c * frames, (c + 1) * frames), the layout read_audio returns.
 */
#ifndef DMX_AUDIO_H
#define DMX_AUDIO_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* AudioInfo (crates/demucs-core/src/audio.rs:60-66). */
typedef struct dmx_audio_info {
    int32_t sample_rate;
    int32_t channels;
    int64_t frames;
} dmx_audio_info;

/* Sample formats a WAV can be written in: sf.write's subtypes PCM_16,
 * PCM_24 and FLOAT (Subtype, audio.rs:366-411). */
enum dmx_wav_subtype { DMX_WAV_PCM16 = 0, DMX_WAV_PCM24 = 1, DMX_WAV_FLOAT = 2 };

/* probe_audio (audio.rs:69-97) for WAV: rate, channels and frame count from
 * the header, without decoding. Read formats: integer PCM of 16, 24 or 32
 * bits and IEEE float of 32 or 64 bits, plain or WAVE_FORMAT_EXTENSIBLE;
 * anything else (8-bit PCM, compressed formats, FLAC) is DMX_ERR_AUDIO. */
int dmx_audio_probe(const char *path, dmx_audio_info *info);

/* read_audio (audio.rs:100-112) for WAV: decodes every frame into `data`
 * (channel-major, capacity >= channels * frames floats, as dmx_audio_probe
 * reports) and fills `info`. Integers scale by 2^-(bits-1), as soundfile
 * hands them to librosa; floats are copied (64-bit ones rounded to 32). */
int dmx_audio_read(const char *path, float *data, int64_t capacity, dmx_audio_info *info);

/* write_wav (audio.rs:464-545): `data` channel-major, `frames` per channel,
 * written interleaved in the given subtype. Integer subtypes round
 * value * 2^(bits-1) half away from zero and clip to the signed range
 * (libsndfile's lrintf + clip, audio.rs:726-731; NaN writes 0). */
int dmx_wav_write(const char *path, int subtype, int32_t sample_rate, int32_t channels, const float *data,
                  int64_t frames);

/* FloatWavWriter (audio.rs:556-669): an IEEE-float WAV written frame by
 * frame, whose RIFF and data sizes are patched by finish. Memory stays
 * O(buffer) whatever the length. */
typedef struct dmx_wav_writer dmx_wav_writer;
int dmx_wav_writer_create(const char *path, int32_t sample_rate, int32_t channels, dmx_wav_writer **out);
/* Appends `frames` interleaved frames (frames * channels floats). */
int dmx_wav_writer_write(dmx_wav_writer *writer, const float *interleaved, int64_t frames);
/* Appends `frames` frames given as `channels` rows of one planar block:
 * channel c's samples start at rows + c * row_stride. */
int dmx_wav_writer_write_planar(dmx_wav_writer *writer, const float *rows, int64_t row_stride, int64_t frames);
int64_t dmx_wav_writer_frames(const dmx_wav_writer *writer);
/* Patches the header and closes the file; frees the writer whatever the
 * outcome (a writer is finished exactly once). */
int dmx_wav_writer_finish(dmx_wav_writer *writer);

/* Comparison (crates/demucs-core/src/fixtures.rs:98-189): element-wise
 * difference of `actual` against `expected`, both n floats. */
typedef struct dmx_comparison {
    int64_t elements;
    float max_abs;           /* max |e - a| */
    int64_t max_abs_index;   /* its index */
    float max_rel;           /* max |e - a| / max(|e|, 1e-6) */
    float mean_abs;          /* mean |e - a| (f64 sum) */
    float reference_max_abs; /* max |e| */
    float reference_rms;     /* sqrt(mean e^2) (f64 sum) */
    float rms_relative_error; /* mean_abs / reference_rms (mean_abs if the reference is silent) */
    float snr_db;            /* -20 log10(rms_relative_error), +inf when it is 0 */
} dmx_comparison;
/* compare (fixtures.rs:152-189), plus the derived metrics of
 * Comparison::rms_relative_error and snr_db (fixtures.rs:133-149). */
int dmx_compare(const float *expected, const float *actual, int64_t n, dmx_comparison *out);

#ifdef __cplusplus
}
#endif

#endif /* DMX_AUDIO_H */
