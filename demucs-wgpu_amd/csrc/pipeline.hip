// pipeline.hip — the chunk loop's device side: global normalisation,
// centred zero-padded chunks (optionally through the shift view), weighted
// overlap-add, the bag's weighted combine, and the final divide/trim/denormalise.
//
// Semantics: scan_norm / apply_norm_inplace (crates/demucs-core/src/demucs/streaming.rs:52-85),
// padded_chunk_mix / padded_chunk_shifted_mix (demucs/mix.rs:552-640),
// OlaRing splice/flush (streaming.rs:96-261), separate_forwarding_emit's
// shift trim and scale (demucs/pipeline.rs:380-515), BagCombineForward
// (api.rs:319-371) and the final `frame * std + mean` (api.rs:720-724).
// Overlapping chunks are added in chunk order per sample, so the sums round
// exactly as the reference's ring does.
#include "common.h"
#include "ops.h"

namespace dmx {
namespace {

constexpr int MAX_GROUP = 64;

struct Spans {
    int64_t start[MAX_GROUP];
    int64_t len[MAX_GROUP];
};

// Channel-mean moments of a stereo mix (2, samples): ref = (l + r) / 2 in f64.
__global__ __launch_bounds__(256) void mix_moments_kernel(const float *__restrict__ mix, int64_t n,
                                                          double *__restrict__ stats) {
    double s = 0.0, q = 0.0;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
        double r = ((double)mix[i] + (double)mix[n + i]) / 2.0;
        s += r;
        q += r * r;
    }
    block_moments_atomic(s, q, stats);
}

// scan_norm's finish: mean, std = sqrt(unbiased var) as f32 + 1e-8.
__device__ __forceinline__ void global_norm(const double *stats, int64_t n, float &mean, float &stdv) {
    double count = (double)n;
    double m = stats[0] / count;
    double var = count > 1.0 ? (stats[1] - stats[0] * stats[0] / count) / (count - 1.0) : 0.0;
    mean = (float)m;
    stdv = (float)sqrt(fmax(var, 0.0)) + 1e-8f;
}

__global__ __launch_bounds__(256) void build_chunks_kernel(const float *__restrict__ mix, int64_t mix_len,
                                                           const double *__restrict__ stats, Spans spans, int64_t seg,
                                                           int64_t view_len, int64_t shift_offset, int64_t max_shift,
                                                           float *__restrict__ out) {
    const int slot = blockIdx.z, ch = blockIdx.y;
    float mean, stdv;
    global_norm(stats, mix_len, mean, stdv);
    const int64_t start = spans.start[slot] - (seg - spans.len[slot]) / 2;
    float *dst = out + ((int64_t)slot * 2 + ch) * seg;
    const float *src = mix + (int64_t)ch * mix_len;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < seg; i += (int64_t)gridDim.x * 256) {
        int64_t vi = start + i;
        float v = 0.0f;
        if (vi >= 0 && vi < view_len) {
            int64_t mi = max_shift > 0 ? shift_offset + vi - max_shift : vi;
            if (mi >= 0 && mi < mix_len) v = (src[mi] - mean) / stdv;
        }
        dst[i] = v;
    }
}

// acc[r][t] += w[t - s0] * out[slot][r][trim + t - s0] for every slot covering t,
// in slot order; sum_w likewise (row 0 of the grid only).
__global__ __launch_bounds__(256) void ola_accumulate_kernel(const float *__restrict__ chunk_out, int group, Spans spans,
                                                             int64_t seg, int rows, int64_t view_len,
                                                             const float *__restrict__ weight, float *__restrict__ acc,
                                                             float *__restrict__ sum_w) {
    const int r = blockIdx.y;
    const int64_t lo = spans.start[0];
    const int64_t hi = spans.start[group - 1] + spans.len[group - 1];
    for (int64_t t = lo + (int64_t)blockIdx.x * 256 + threadIdx.x; t < hi; t += (int64_t)gridDim.x * 256) {
        float a = acc[(int64_t)r * view_len + t];
        float ws = r == 0 ? sum_w[t] : 0.0f;
        for (int slot = 0; slot < group; ++slot) {
            int64_t s0 = spans.start[slot], cl = spans.len[slot];
            int64_t u = t - s0;
            if (u < 0 || u >= cl) continue;
            int64_t trim = (seg - cl) / 2;
            float w = weight[u];
            a += w * chunk_out[((int64_t)slot * rows + r) * seg + trim + u];
            ws += w;
        }
        acc[(int64_t)r * view_len + t] = a;
        if (r == 0) sum_w[t] = ws;
    }
}

// Output samples t in [lo, hi): frame = acc / sum_w at view index t + trim;
// then either
//   mode 0: stems = (frame * scale) * std + mean           (the only pass)
//   mode 1: stems += frame                                 (a pass of several, not the last)
//   mode 2: stems = ((stems + frame) * scale) * std + mean (the last pass of several)
// which rounds as the reference's sum over passes, * 1/shifts, * std + mean.
__global__ __launch_bounds__(256) void ola_finish_kernel(const float *__restrict__ acc, const float *__restrict__ sum_w,
                                                         int64_t view_len, int64_t trim, int64_t lo, int64_t hi,
                                                         int64_t samples, const double *__restrict__ stats,
                                                         int64_t mix_len, float scale, int mode,
                                                         float *__restrict__ stems,
                                                         const uint8_t *__restrict__ row_mask, int channels) {
    const int r = blockIdx.y;
    if (row_mask && !row_mask[r / channels]) return;
    float mean, stdv;
    global_norm(stats, mix_len, mean, stdv);
    for (int64_t t = lo + (int64_t)blockIdx.x * 256 + threadIdx.x; t < hi; t += (int64_t)gridDim.x * 256) {
        float *dst = stems + (int64_t)r * samples + t;
        int64_t tv = t + trim;
        float frame = acc[(int64_t)r * view_len + tv] / sum_w[tv];
        if (mode == 0)
            *dst = (frame * scale) * stdv + mean;
        else if (mode == 1)
            *dst += frame;
        else
            *dst = ((*dst + frame) * scale) * stdv + mean;
    }
}

// combined[b][s] (+)= net_out[b][s] * w[s] over requested sources (w[s] = 0 skips).
__global__ __launch_bounds__(256) void bag_accumulate_kernel(const float *__restrict__ net_out, int sources,
                                                             int64_t per_source, const float *__restrict__ weights,
                                                             float *__restrict__ combined, int first) {
    const int bs = blockIdx.y, s = bs % sources;
    const float w = weights[s];
    if (w == 0.0f) return;
    const int64_t base = (int64_t)bs * per_source;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < per_source; i += (int64_t)gridDim.x * 256) {
        float v = net_out[base + i] * w;
        combined[base + i] = first ? v : combined[base + i] + v;
    }
}

__global__ __launch_bounds__(256) void bag_divide_kernel(float *__restrict__ combined, int sources, int64_t per_source,
                                                         const float *__restrict__ totals) {
    const int bs = blockIdx.y, s = bs % sources;
    const float t = totals[s];
    if (t == 0.0f) return;
    const int64_t base = (int64_t)bs * per_source;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < per_source; i += (int64_t)gridDim.x * 256)
        combined[base + i] = combined[base + i] / t;
}

unsigned gcap(int64_t n, int64_t cap) { return (unsigned)std::max<int64_t>(1, std::min<int64_t>(ceil_div(n, 256), cap)); }

Spans make_spans(int group, const int64_t *starts, const int64_t *lengths) {
    DMX_REQUIRE(group > 0 && group <= MAX_GROUP, "chunk group size out of range");
    Spans sp{};
    for (int i = 0; i < group; ++i) {
        sp.start[i] = starts[i];
        sp.len[i] = lengths[i];
    }
    return sp;
}

}  // namespace

void mix_moments(hipStream_t s, const float *mix, int64_t samples, double *stats) {
    zero_doubles(s, stats, 2);
    hipLaunchKernelGGL(mix_moments_kernel, dim3(gcap(samples, 1024)), dim3(256), 0, s, mix, samples, stats);
    DMX_LAUNCH_CHECK();
}

void build_chunks(hipStream_t s, const float *mix, int64_t mix_len, const double *stats, int group,
                  const int64_t *starts, const int64_t *lengths, int64_t seg, int64_t view_len, int64_t shift_offset,
                  int64_t max_shift, float *out) {
    require_ptrs({mix, stats, out}, "build_chunks");
    Spans sp = make_spans(group, starts, lengths);
    hipLaunchKernelGGL(build_chunks_kernel, dim3(gcap(seg, 512), 2, (unsigned)group), dim3(256), 0, s, mix, mix_len,
                       stats, sp, seg, view_len, shift_offset, max_shift, out);
    DMX_LAUNCH_CHECK();
}

void ola_accumulate(hipStream_t s, const float *chunk_out, int group, const int64_t *starts, const int64_t *lengths,
                    int64_t seg, int rows, int64_t view_len, const float *weight, float *acc, float *sum_w) {
    require_ptrs({chunk_out, weight, acc, sum_w}, "ola_accumulate");
    Spans sp = make_spans(group, starts, lengths);
    for (int i = 0; i < group; ++i)
        DMX_REQUIRE(starts[i] >= 0 && lengths[i] > 0 && lengths[i] <= seg && starts[i] + lengths[i] <= view_len,
                    "ola_accumulate: chunk span outside the view");
    int64_t span =starts[group - 1] + lengths[group - 1] - starts[0];
    // Row 0 also owns sum_w; every row reads only its own acc row.
    hipLaunchKernelGGL(ola_accumulate_kernel, dim3(gcap(span, 2048), (unsigned)rows), dim3(256), 0, s, chunk_out, group,
                       sp, seg, rows, view_len, weight, acc, sum_w);
    DMX_LAUNCH_CHECK();
}

void ola_finish(hipStream_t s, const float *acc, const float *sum_w, int rows, int64_t view_len, int64_t trim,
                int64_t lo, int64_t hi, int64_t samples, const double *stats, float scale, int mode, float *stems,
                const uint8_t *row_mask) {
    // `stats` are the mix moments; samples is the mix length they were taken over.
    require_ptrs({acc, sum_w, stats, stems}, "ola_finish");
    DMX_REQUIRE(mode >= 0 && mode <= 2, "ola_finish: unknown mode");
    DMX_REQUIRE(0 <= lo && lo <= hi && hi <= samples && hi + trim <= view_len, "ola_finish: range outside the view");
    if (hi == lo) return;
    hipLaunchKernelGGL(ola_finish_kernel, dim3(gcap(hi - lo, 2048), (unsigned)rows), dim3(256), 0, s, acc, sum_w,
                       view_len, trim, lo, hi, samples, stats, samples, scale, mode, stems, row_mask, 2);
    DMX_LAUNCH_CHECK();
}

void bag_accumulate(hipStream_t s, const float *net_out, int64_t group_batch, int sources, int64_t per_source,
                    const float *weights, float *combined, int first) {
    hipLaunchKernelGGL(bag_accumulate_kernel, dim3(gcap(per_source, 1024), (unsigned)(group_batch * sources)),
                       dim3(256), 0, s, net_out, sources, per_source, weights, combined, first);
    DMX_LAUNCH_CHECK();
}

void bag_divide(hipStream_t s, float *combined, int64_t group_batch, int sources, int64_t per_source,
                const float *totals) {
    hipLaunchKernelGGL(bag_divide_kernel, dim3(gcap(per_source, 1024), (unsigned)(group_batch * sources)), dim3(256), 0,
                       s, combined, sources, per_source, totals);
    DMX_LAUNCH_CHECK();
}

}  // namespace dmx
