// audio.cpp — WAV files and the comparison metric behind include/dmx_audio.h.
//
// Host-only. A WAV file is a RIFF container: "RIFF" <size> "WAVE", then
// chunks of <4-byte id><u32 little-endian size><body, padded to even size>.
// The reader walks the chunks for "fmt " and "data" (anything between them,
// such as soundfile's "fact" and "PEAK", is skipped) and decodes the PCM in
// windows straight into a channel-major buffer. The formats read are those
// of crates/demucs-core/src/audio.rs:315-357 (PCM 16/24/32, float 32/64);
// the writer emits the three subtypes of audio.rs:464-545.
#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <limits>
#include <memory>
#include <string>
#include <vector>

#include "../../include/dmx.h"
#include "../../include/dmx_audio.h"
#include "status.h"

namespace dmx {
namespace {

constexpr uint16_t TAG_PCM = 1, TAG_FLOAT = 3, TAG_EXTENSIBLE = 0xFFFE;

[[noreturn]] void audio_error(const std::string &path, const std::string &what) {
    throw_error(DMX_ERR_AUDIO, path + ": " + what);
}

uint16_t le16(const unsigned char *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
uint32_t le32(const unsigned char *p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

// An open file that closes itself.
struct File {
    FILE *f = nullptr;
    std::string path;
    File(const char *p, const char *mode) : path(p ? p : "") {
        if (!p) throw_error(DMX_ERR_ARGUMENT, "null path");
        f = std::fopen(p, mode);
        if (!f) throw_error(DMX_ERR_IO, "io error on " + path + ": " + std::strerror(errno));
    }
    ~File() {
        if (f) std::fclose(f);
    }
    File(const File &) = delete;
    File &operator=(const File &) = delete;
    // Reads exactly n bytes; false at a clean end of file before any byte.
    bool read(void *dst, size_t n, const char *what) {
        const size_t got = std::fread(dst, 1, n, f);
        if (got == n) return true;
        if (got == 0 && std::feof(f)) return false;
        audio_error(path, std::string("file ends inside the ") + what);
    }
    void skip(uint64_t n) {
        if (n && std::fseek(f, (long)n, SEEK_CUR) != 0) audio_error(path, "cannot seek past a chunk");
    }
    void write(const void *src, size_t n) {
        if (std::fwrite(src, 1, n, f) != n) throw_error(DMX_ERR_IO, "io error on " + path + ": " + std::strerror(errno));
    }
};

// What the header says about the samples, and where they are.
struct WavLayout {
    int encoding = 0;  // TAG_PCM or TAG_FLOAT after resolving EXTENSIBLE
    int bits = 0;
    int channels = 0;
    uint32_t rate = 0;
    uint64_t data_bytes = 0;
    long data_offset = 0;
    int64_t frames() const { return (int64_t)(data_bytes / ((uint64_t)channels * (uint64_t)(bits / 8))); }
};

// Parses the chunk list up to the start of the "data" payload and leaves
// the file positioned there.
WavLayout scan(File &file) {
    unsigned char riff[12];
    if (!file.read(riff, 12, "RIFF header") || std::memcmp(riff, "RIFF", 4) != 0 ||
        std::memcmp(riff + 8, "WAVE", 4) != 0)
        audio_error(file.path, "not a RIFF/WAVE file (only uncompressed WAV is read)");
    WavLayout w;
    bool have_fmt = false;
    int tag = 0, block_align = 0;
    for (;;) {
        unsigned char head[8];
        if (!file.read(head, 8, "chunk header")) break;
        const uint32_t size = le32(head + 4);
        const uint64_t padded = (uint64_t)size + (size & 1u);
        if (std::memcmp(head, "fmt ", 4) == 0) {
            if (size < 16) audio_error(file.path, "fmt chunk shorter than 16 bytes");
            std::vector<unsigned char> body(size);
            file.read(body.data(), size, "fmt chunk");
            if (size & 1u) file.skip(1);
            tag = le16(&body[0]);
            w.channels = le16(&body[2]);
            w.rate = le32(&body[4]);
            block_align = le16(&body[12]);
            w.bits = le16(&body[14]);
            if (tag == TAG_EXTENSIBLE) {
                // cbSize (2), valid bits (2), channel mask (4), sub-format GUID
                // whose first two bytes are the format tag.
                if (size < 40) audio_error(file.path, "WAVE_FORMAT_EXTENSIBLE fmt chunk shorter than 40 bytes");
                tag = le16(&body[24]);
            }
            have_fmt = true;
        } else if (std::memcmp(head, "data", 4) == 0) {
            if (!have_fmt) audio_error(file.path, "data chunk before the fmt chunk");
            w.data_bytes = size;
            w.data_offset = std::ftell(file.f);
            break;
        } else {
            file.skip(padded);
        }
    }
    if (!have_fmt) audio_error(file.path, "missing fmt chunk");
    if (w.data_offset == 0) audio_error(file.path, "missing data chunk");
    if (w.channels <= 0) audio_error(file.path, "zero channels");
    const bool pcm_ok = tag == TAG_PCM && (w.bits == 16 || w.bits == 24 || w.bits == 32);
    const bool float_ok = tag == TAG_FLOAT && (w.bits == 32 || w.bits == 64);
    if (!pcm_ok && !float_ok)
        audio_error(file.path, "unsupported WAV encoding (format tag " + std::to_string(tag) + ", " +
                                   std::to_string(w.bits) + " bits per sample)");
    w.encoding = tag;
    const int frame_bytes = w.channels * (w.bits / 8);
    if (block_align != frame_bytes)
        audio_error(file.path, "block align " + std::to_string(block_align) + " does not match " +
                                   std::to_string(w.channels) + " channels of " + std::to_string(w.bits) + " bits");
    if (w.data_bytes % (uint64_t)frame_bytes != 0)
        audio_error(file.path, "data chunk of " + std::to_string(w.data_bytes) + " bytes is not a whole number of " +
                                   std::to_string(frame_bytes) + "-byte frames");
    return w;
}

// One sample of the interleaved payload as float, scaled like soundfile.
inline float decode_sample(const unsigned char *p, int encoding, int bits) {
    if (encoding == TAG_FLOAT) {
        if (bits == 32) {
            float v;
            std::memcpy(&v, p, 4);
            return v;
        }
        double v;
        std::memcpy(&v, p, 8);
        return (float)v;
    }
    switch (bits) {
        case 16:
            return (float)(int16_t)le16(p) * (1.0f / 32768.0f);
        case 24: {
            // Sign-extend the 24-bit two's complement value through the top byte.
            const int32_t v = (int32_t)((uint32_t)p[0] << 8 | (uint32_t)p[1] << 16 | (uint32_t)p[2] << 24) >> 8;
            return (float)v * (1.0f / 8388608.0f);
        }
        default:
            return (float)(int32_t)le32(p) * (1.0f / 2147483648.0f);
    }
}

// round(value * 2^(bits-1)) half away from zero, clipped to the signed range.
inline int32_t quantize(float value, int bits) {
    const float scale = (float)(1LL << (bits - 1));
    const float lo = -scale, hi = scale - 1.0f;
    float v = std::round(value * scale);
    if (std::isnan(v)) return 0;
    v = v < lo ? lo : v > hi ? hi : v;
    return (int32_t)v;
}

void put_header(File &file, uint16_t tag, int channels, uint32_t rate, int bytes_per_sample, uint32_t data_bytes) {
    unsigned char h[44];
    auto put16 = [&](int at, uint32_t v) {
        h[at] = (unsigned char)v;
        h[at + 1] = (unsigned char)(v >> 8);
    };
    auto put32 = [&](int at, uint32_t v) {
        for (int i = 0; i < 4; ++i) h[at + i] = (unsigned char)(v >> (8 * i));
    };
    const uint32_t align = (uint32_t)channels * (uint32_t)bytes_per_sample;
    std::memcpy(h, "RIFF", 4);
    put32(4, 36u + data_bytes);
    std::memcpy(h + 8, "WAVEfmt ", 8);
    put32(16, 16);
    put16(20, tag);
    put16(22, (uint32_t)channels);
    put32(24, rate);
    put32(28, rate * align);
    put16(32, align);
    put16(34, (uint32_t)bytes_per_sample * 8);
    std::memcpy(h + 36, "data", 4);
    put32(40, data_bytes);
    file.write(h, 44);
}

// Classic RIFF sizes are 32-bit: 36 header bytes plus the payload must fit.
uint32_t checked_payload(const std::string &path, int64_t frames, int channels, int bytes_per_sample) {
    const long double bytes = (long double)frames * channels * bytes_per_sample;
    if (bytes + 36 > (long double)std::numeric_limits<uint32_t>::max())
        audio_error(path, "WAV payload of " + std::to_string((long long)bytes) + " bytes exceeds RIFF's 4 GiB");
    return (uint32_t)bytes;
}

constexpr int64_t WINDOW_FRAMES = 8192;

}  // namespace
}  // namespace dmx

struct dmx_wav_writer {
    dmx::File file;
    int channels;
    int64_t frames = 0;
    std::vector<unsigned char> buf;
    dmx_wav_writer(const char *path, int ch) : file(path, "wb"), channels(ch) {}
};

using namespace dmx;

extern "C" {

int dmx_audio_probe(const char *path, dmx_audio_info *info) {
    return guarded([&] {
        if (!info) throw_error(DMX_ERR_ARGUMENT, "null info");
        File file(path, "rb");
        const WavLayout w = scan(file);
        *info = {(int32_t)w.rate, (int32_t)w.channels, w.frames()};
    });
}

int dmx_audio_read(const char *path, float *data, int64_t capacity, dmx_audio_info *info) {
    return guarded([&] {
        if (!data || !info) throw_error(DMX_ERR_ARGUMENT, "null argument");
        File file(path, "rb");
        const WavLayout w = scan(file);
        const int64_t frames = w.frames();
        if (capacity < frames * w.channels)
            throw_error(DMX_ERR_SHAPE, file.path + ": " + std::to_string(frames * w.channels) +
                                           " samples do not fit a buffer of " + std::to_string(capacity));
        const int sample_bytes = w.bits / 8, frame_bytes = w.channels * sample_bytes;
        std::vector<unsigned char> window((size_t)std::min<int64_t>(frames, WINDOW_FRAMES) * frame_bytes + 1);
        for (int64_t at = 0; at < frames; at += WINDOW_FRAMES) {
            const int64_t n = std::min<int64_t>(WINDOW_FRAMES, frames - at);
            if (!file.read(window.data(), (size_t)(n * frame_bytes), "data chunk") && n > 0)
                audio_error(file.path, "file ends inside the data chunk");
            const unsigned char *p = window.data();
            for (int64_t i = 0; i < n; ++i)
                for (int c = 0; c < w.channels; ++c, p += sample_bytes)
                    data[(int64_t)c * frames + at + i] = decode_sample(p, w.encoding, w.bits);
        }
        *info = {(int32_t)w.rate, (int32_t)w.channels, frames};
    });
}

int dmx_wav_write(const char *path, int subtype, int32_t sample_rate, int32_t channels, const float *data,
                  int64_t frames) {
    return guarded([&] {
        if (!data && frames > 0) throw_error(DMX_ERR_ARGUMENT, "null data");
        if (subtype < DMX_WAV_PCM16 || subtype > DMX_WAV_FLOAT) throw_error(DMX_ERR_ARGUMENT, "unknown WAV subtype");
        if (channels <= 0) throw_error(DMX_ERR_AUDIO, "cannot write zero channels");
        if (frames < 0 || sample_rate <= 0) throw_error(DMX_ERR_ARGUMENT, "negative frame count or rate");
        const int bps = subtype == DMX_WAV_PCM16 ? 2 : subtype == DMX_WAV_PCM24 ? 3 : 4;
        File file(path, "wb");
        const uint32_t payload = checked_payload(file.path, frames, channels, bps);
        put_header(file, subtype == DMX_WAV_FLOAT ? TAG_FLOAT : TAG_PCM, channels, (uint32_t)sample_rate, bps, payload);
        std::vector<unsigned char> out((size_t)std::min<int64_t>(frames, WINDOW_FRAMES) * channels * bps + 1);
        for (int64_t at = 0; at < frames; at += WINDOW_FRAMES) {
            const int64_t n = std::min<int64_t>(WINDOW_FRAMES, frames - at);
            unsigned char *p = out.data();
            for (int64_t i = 0; i < n; ++i)
                for (int c = 0; c < channels; ++c) {
                    const float v = data[(int64_t)c * frames + at + i];
                    if (subtype == DMX_WAV_FLOAT) {
                        std::memcpy(p, &v, 4);
                    } else {
                        const uint32_t q = (uint32_t)quantize(v, bps * 8);
                        for (int b = 0; b < bps; ++b) p[b] = (unsigned char)(q >> (8 * b));
                    }
                    p += bps;
                }
            file.write(out.data(), (size_t)(p - out.data()));
        }
        if (std::fflush(file.f) != 0) throw_error(DMX_ERR_IO, "io error on " + file.path + ": " + std::strerror(errno));
    });
}

int dmx_wav_writer_create(const char *path, int32_t sample_rate, int32_t channels, dmx_wav_writer **out) {
    return guarded([&] {
        if (!out) throw_error(DMX_ERR_ARGUMENT, "null out");
        *out = nullptr;
        if (channels <= 0) throw_error(DMX_ERR_AUDIO, "cannot write zero channels");
        if (sample_rate <= 0) throw_error(DMX_ERR_ARGUMENT, "sample rate must be positive");
        auto *w = new dmx_wav_writer(path, channels);
        try {
            put_header(w->file, TAG_FLOAT, channels, (uint32_t)sample_rate, 4, 0);  // sizes patched by finish
        } catch (...) {
            delete w;
            throw;
        }
        *out = w;
    });
}

int dmx_wav_writer_write(dmx_wav_writer *w, const float *interleaved, int64_t frames) {
    return guarded([&] {
        if (!w || (!interleaved && frames > 0)) throw_error(DMX_ERR_ARGUMENT, "null argument");
        if (frames < 0) throw_error(DMX_ERR_ARGUMENT, "negative frame count");
        checked_payload(w->file.path, w->frames + frames, w->channels, 4);
        w->file.write(interleaved, (size_t)frames * (size_t)w->channels * sizeof(float));
        w->frames += frames;
    });
}

int dmx_wav_writer_write_planar(dmx_wav_writer *w, const float *rows, int64_t row_stride, int64_t frames) {
    return guarded([&] {
        if (!w || (!rows && frames > 0)) throw_error(DMX_ERR_ARGUMENT, "null argument");
        if (frames < 0 || (w->channels > 1 && row_stride < frames))
            throw_error(DMX_ERR_ARGUMENT, "rows overlap or the frame count is negative");
        checked_payload(w->file.path, w->frames + frames, w->channels, 4);
        const int C = w->channels;
        std::vector<float> inter((size_t)std::min<int64_t>(frames, WINDOW_FRAMES) * C + 1);
        for (int64_t at = 0; at < frames; at += WINDOW_FRAMES) {
            const int64_t n = std::min<int64_t>(WINDOW_FRAMES, frames - at);
            for (int c = 0; c < C; ++c) {
                const float *src = rows + (int64_t)c * row_stride + at;
                for (int64_t i = 0; i < n; ++i) inter[(size_t)(i * C + c)] = src[i];
            }
            w->file.write(inter.data(), (size_t)n * C * sizeof(float));
        }
        w->frames += frames;
    });
}

int64_t dmx_wav_writer_frames(const dmx_wav_writer *w) { return w ? w->frames : 0; }

int dmx_wav_writer_finish(dmx_wav_writer *w) {
    return guarded([&] {
        if (!w) throw_error(DMX_ERR_ARGUMENT, "null writer");
        std::unique_ptr<dmx_wav_writer> own(w);
        const uint32_t payload = checked_payload(w->file.path, w->frames, w->channels, 4);
        unsigned char v[4];
        auto patch = [&](long at, uint32_t x) {
            for (int i = 0; i < 4; ++i) v[i] = (unsigned char)(x >> (8 * i));
            if (std::fseek(w->file.f, at, SEEK_SET) != 0) throw_error(DMX_ERR_IO, "io error on " + w->file.path);
            w->file.write(v, 4);
        };
        patch(4, 36u + payload);
        patch(40, payload);
        if (std::fflush(w->file.f) != 0)
            throw_error(DMX_ERR_IO, "io error on " + w->file.path + ": " + std::strerror(errno));
    });
}

int dmx_compare(const float *expected, const float *actual, int64_t n, dmx_comparison *out) {
    return guarded([&] {
        if (!out || ((!expected || !actual) && n > 0)) throw_error(DMX_ERR_ARGUMENT, "null argument");
        if (n < 0) throw_error(DMX_ERR_ARGUMENT, "negative length");
        dmx_comparison r{};
        r.elements = n;
        double sum_abs = 0.0, sum_sq = 0.0;
        for (int64_t i = 0; i < n; ++i) {
            const float e = expected[i], a = actual[i];
            const float d = std::fabs(e - a);
            if (d > r.max_abs) {
                r.max_abs = d;
                r.max_abs_index = i;
            }
            const float rel = d / std::max(std::fabs(e), 1e-6f);
            if (rel > r.max_rel) r.max_rel = rel;
            sum_abs += (double)d;
            sum_sq += (double)e * (double)e;
            r.reference_max_abs = std::max(r.reference_max_abs, std::fabs(e));
        }
        if (n > 0) {
            r.mean_abs = (float)(sum_abs / (double)n);
            r.reference_rms = (float)std::sqrt(sum_sq / (double)n);
        }
        r.rms_relative_error = r.reference_rms > 0.0f ? r.mean_abs / r.reference_rms : r.mean_abs;
        r.snr_db = r.rms_relative_error <= 0.0f ? std::numeric_limits<float>::infinity()
                                                : -20.0f * std::log10(r.rms_relative_error);
        *out = r;
    });
}

}  // extern "C"
