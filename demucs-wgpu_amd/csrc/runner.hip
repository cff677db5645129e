// runner.hip — the HTDemucs segment forward on one MI355X, and the C-ABI of
// include/dmx.h around it.
//
// The forward walks the graph of `Htdemucs::forward`
// (crates/demucs-core/src/demucs/host.rs:202-520) with one fused launch per
// op group; every intermediate lives in HBM in the reference's own layout
// ((b, c, f, t) for the branches, (b, tokens, c) inside the transformer), so a
// traced activation needs no conversion. Intermediates come from the
// stream-ordered pool (hipMallocAsync / hipFreeAsync on the runner's stream),
// which recycles them without host synchronisation.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/dmx.h"
#include "common.h"
#include "ops.h"
#include "staging.h"

namespace dmx {
namespace {


// Caching device allocator, one free list per stream. All work that touches a
// block is enqueued on the stream it was taken for, so a block returned to the
// list can be handed out again at once: any later use is ordered after every
// earlier one on that stream. Blocks go back to the device only when the
// stream's runner is destroyed.
class StreamPool {
  public:
    static StreamPool &instance() {
        static StreamPool pool;
        return pool;
    }
    void *take(hipStream_t s, size_t bytes) {
        bytes = round_up(bytes);
        {
            std::lock_guard<std::mutex> lock(mu_);
            auto &free = free_[s];
            auto it = free.lower_bound(bytes);
            if (it != free.end() && it->first <= 2 * bytes + (2u << 20)) {
                void *p = it->second;
                sizes_[p] = it->first;
                free.erase(it);
                return p;
            }
        }
        void *p = nullptr;
        hipError_t e = hipMalloc(&p, bytes);
        if (e != hipSuccess) {
            // Release this stream's cached blocks and try once more.
            trim(s);
            DMX_HIP(hipMalloc(&p, bytes));
        }
        std::lock_guard<std::mutex> lock(mu_);
        sizes_[p] = bytes;
        owner_[p] = s;
        return p;
    }
    void give(hipStream_t s, void *p) {
        std::lock_guard<std::mutex> lock(mu_);
        auto it = sizes_.find(p);
        if (it == sizes_.end()) return;
        free_[s].emplace(it->second, p);
        sizes_.erase(it);
    }
    // Frees every cached block of `s` (after the stream has drained).
    void trim(hipStream_t s) {
        (void)hipStreamSynchronize(s);
        std::lock_guard<std::mutex> lock(mu_);
        auto &free = free_[s];
        for (auto &kv : free) {
            (void)hipFree(kv.second);
            owner_.erase(kv.second);
        }
        free.clear();
    }

  private:
    static size_t round_up(size_t b) {
        const size_t g = b >= (1u << 20) ? (1u << 20) : 512;
        return (std::max<size_t>(b, 1) + g - 1) / g * g;
    }
    std::mutex mu_;
    std::map<hipStream_t, std::multimap<size_t, void *>> free_;
    std::map<void *, size_t> sizes_;     // blocks in use -> size
    std::map<void *, hipStream_t> owner_;
};

// A device buffer from the stream's cache, returned to it on scope exit.
struct DBuf {
    hipStream_t s = nullptr;
    void *p = nullptr;
    size_t bytes = 0;
    DBuf() = default;
    DBuf(hipStream_t stream, size_t n_bytes) : s(stream), bytes(n_bytes) {
        if (bytes) p = StreamPool::instance().take(s, bytes);
    }
    DBuf(const DBuf &) = delete;
    DBuf &operator=(const DBuf &) = delete;
    DBuf(DBuf &&o) noexcept : s(o.s), p(o.p), bytes(o.bytes) { o.p = nullptr; }
    DBuf &operator=(DBuf &&o) noexcept {
        if (this != &o) {
            release();
            s = o.s;
            p = o.p;
            bytes = o.bytes;
            o.p = nullptr;
        }
        return *this;
    }
    ~DBuf() { release(); }
    void release() {
        if (p) StreamPool::instance().give(s, p);
        p = nullptr;
    }
    float *f() const { return static_cast<float *>(p); }
    double *d() const { return static_cast<double *>(p); }
};

DBuf fbuf(hipStream_t s, int64_t n) { return DBuf(s, (size_t)std::max<int64_t>(n, 1) * sizeof(float)); }
// Plane stride (bf16 elements) of an n-element operand: whole 16-byte rows.
int64_t plane_stride(int64_t n) { return (n + 7) / 8 * 8; }
// A buffer for n elements either as fp32 or as P bf16 planes.
DBuf obuf(hipStream_t s, int64_t n, int P) {
    return DBuf(s, std::max<size_t>((size_t)std::max<int64_t>(n, 1) * sizeof(float),
                                    (size_t)plane_stride(n) * P * sizeof(unsigned short)));
}
Planes planes_in(const DBuf &b, int64_t n, int P) {
    return Planes{static_cast<unsigned short *>(b.p), plane_stride(n), P};
}
DBuf dbuf(hipStream_t s, int64_t n) { return DBuf(s, (size_t)std::max<int64_t>(n, 1) * sizeof(double)); }

struct Trace {
    dmx_trace_wants_fn wants = nullptr;
    dmx_trace_record_fn record = nullptr;
    void *user = nullptr;
};

struct DConvW {
    const float *w1, *b1, *n1w, *n1b, *w2, *b2, *n2w, *n2b, *gamma;
    int hidden;
    const float *w1_gemm;  // w1 in GEMM order (conv_gemm_weights)
    const float *w1_t;     // w1 as (C*3, H) for the narrow path (dconv_w1_transposed), or null
    const double *gram;    // conv2 folded for its moments from a Gram matrix (dconv_gram_weights), or null
};

struct LayerW {
    const float *conv_w = nullptr, *conv_b = nullptr, *rw = nullptr, *rb = nullptr;
    const float *rw_wino = nullptr;  // decoder rewrite as Winograd U (winograd_weights), or null
    int cin = 0, cout = 0;
    DConvW dconv[2];
};

struct TLayerW {
    bool cross;
    const float *in_w, *in_b, *out_w, *out_b, *w1, *b1, *w2, *b2;
    const float *n1w, *n1b, *n2w, *n2b, *n3w, *n3b, *now_, *nob, *g1, *g2;
    // The four linear weights as bf16 planes, when the runner's linears run
    // on planes (count 0 otherwise).
    Planes in_wp, out_wp, w1p, w2p;
};

}  // namespace
}  // namespace dmx

namespace dmx {
namespace {
// Pinned staging of one SegmentForward group in flight: the caller's mix is
// copied into `in`, the stems come back into `out`. Slots belong to the
// runner and are reused; a slot grows only when a larger group comes.
struct PendingSlot {
    float *in = nullptr, *out = nullptr;
    size_t in_cap = 0, out_cap = 0;  // floats
    hipEvent_t done = nullptr;       // the group's stems are in `out`
    bool busy = false;
};
}  // namespace
}  // namespace dmx

struct dmx_pending {
    dmx_runner *runner = nullptr;
    int slot = -1;
    size_t count = 0;  // floats of stems
};

struct dmx_runner {
    dmx_config cfg{};
    int device = 0;
    int precision = 0;
    int planes = 0;  // bf16 planes per operand of the transformer linears (0: fp32 MFMA)
    hipStream_t stream = nullptr;
    // The waveform branch runs on its own stream beside the spectral one
    // (all default priority); fork/join are event waits on the GPU.
    hipStream_t side = nullptr;
    // A second (main, side) pair: the device separation runs every other
    // chunk group on it, so two groups' forwards overlap.
    hipStream_t stream_b = nullptr, side_b = nullptr;
    hipEvent_t ev_fork = nullptr, ev_join = nullptr, ev_lane = nullptr;
    // Set while the chunk loop wants the forward to mark, on its main stream,
    // the point the other lane's next group starts from (ev_mid): 1 = before
    // the transformer, 2 = after it, 10 + i = after encoder level i, 20 + i =
    // after frequency decoder level i, 30 + i = after transformer layer i.
    hipEvent_t ev_mid = nullptr;
    int mark_mid = 0;
    std::string tag;
    int64_t training_length = 0;
    int hop = 0, pre_channels = 0, tch = 0, hidden = 0, freq_emb_rows = 0;

    void *weight_mem = nullptr;
    std::map<std::string, float *> w;
    std::vector<dmx::LayerW> enc, tenc, dec, tdec;  // decoders in execution order
    float *freq_emb = nullptr;                      // (rows, channels) x emb_scale
    std::vector<dmx::TLayerW> layers, layers_t;
    float *twiddles = nullptr;                      // nfft/2 complex + nfft window
    std::map<std::pair<int64_t, int64_t>, float *> pos2d;  // (freqs, frames) -> (T*F, D)
    std::map<int64_t, float *> pos1d;                       // length -> (L, D)
    std::map<std::pair<int64_t, double>, float *> ola_weights;  // (segment, power) -> (seg)
    std::vector<void *> owned;                              // device blocks freed at destroy
    float *eye = nullptr;                                   // (D, D) identity + D zeros
    dmx::Trace trace;
    std::vector<hipEvent_t> marks;          // per chunk group of a separation (mark_event)
    dmx::PinnedBuffer staging;              // dmx_separate's mix and stems in pinned memory
    dmx::PinnedRing ring;                   // its staging for calls too large for `staging`
    std::vector<hipEvent_t> xfer;           // per readback block of dmx_separate (xfer_event)
    std::vector<dmx::PendingSlot> pending;  // staging of dmx_forward_start / collect
    int next_lane = 0;                      // lane of the next dmx_forward_start
};

namespace dmx {
namespace {

float *dev(dmx_runner &r, const std::string &name) {
    auto it = r.w.find(name);
    if (it == r.w.end()) throw_error(DMX_ERR_MISSING_WEIGHT, "weight `" + name + "` not found in checkpoint");
    return it->second;
}

float *upload(dmx_runner &r, const std::vector<float> &host) {
    void *p = nullptr;
    DMX_HIP(hipMalloc(&p, std::max<size_t>(host.size(), 1) * sizeof(float)));
    r.owned.push_back(p);
    if (!host.empty()) DMX_HIP(hipMemcpy(p, host.data(), host.size() * sizeof(float), hipMemcpyHostToDevice));
    return static_cast<float *>(p);
}

bool wants(const dmx_runner &r, const std::string &name) {
    return r.trace.record && (!r.trace.wants || r.trace.wants(name.c_str(), r.trace.user));
}

void record(dmx_runner &r, const std::string &name, const float *d, std::initializer_list<int64_t> shape) {
    if (!wants(r, name)) return;
    std::vector<int64_t> s(shape);
    int64_t n = 1;
    for (int64_t v : s) n *= v;
    std::vector<float> host((size_t)n);
    DMX_HIP(hipStreamSynchronize(r.stream));
    DMX_HIP(hipMemcpy(host.data(), d, (size_t)n * sizeof(float), hipMemcpyDeviceToHost));
    r.trace.record(name.c_str(), s.data(), (int32_t)s.size(), host.data(), r.trace.user);
}

// The two branches of the forward (spectral on `s`, waveform on `t`). They
// only meet at the transformer's cross layers and at the final sum, so the
// waveform work runs on the runner's side stream between fork() (t waits for
// everything enqueued on s so far) and join() (s waits for everything on t).
// Buffer rule: a buffer that work on both streams touches comes from s's
// pool, is taken before the fork and released after the join; a buffer only
// t's work touches comes from t's pool. With a trace sink the whole forward
// stays on s (record() reads activations in stream order); so it does with
// DMX_SINGLE_STREAM=1 in the environment, which gives per-kernel profiles
// without overlap.
bool single_stream_env() {
    static const bool on = [] {
        const char *v = std::getenv("DMX_SINGLE_STREAM");
        return v && v[0] == '1';
    }();
    return on;
}
struct Branches {
    dmx_runner &r;
    hipStream_t s, t;
    Branches(dmx_runner &runner, hipStream_t main)
        : r(runner), s(main),
          t(runner.trace.record || !runner.side || single_stream_env() ? main
            : main == runner.stream_b                                   ? runner.side_b
                                                                        : runner.side) {}
    void fork() {
        if (t == s) return;
        DMX_HIP(hipEventRecord(r.ev_fork, s));
        DMX_HIP(hipStreamWaitEvent(t, r.ev_fork, 0));
    }
    void join() {
        if (t == s) return;
        DMX_HIP(hipEventRecord(r.ev_join, t));
        DMX_HIP(hipStreamWaitEvent(s, r.ev_join, 0));
    }
};

// The configurations the kernels are written for; anything else is refused
// with the UnsupportedModel kind rather than computed wrongly (the same set
// HtdemucsConfig::validate admits, crates/demucs-core/src/demucs/config.rs:239-273).
void validate(const dmx_config &c) {
    // The spectral branch keeps more than one bin through every encoder level
    // (a level whose input has at most kernel_size bins would merge the two
    // branches inside the encoder, which this backend does not build).
    bool bins_survive = true;
    for (int i = 0, f = c.nfft / 2; i < c.depth; ++i) {
        if (f > 1 && f <= c.kernel_size) bins_survive = false;
        if (f > 1) f /= std::max(c.stride, 1);
    }
    const struct {
        bool ok;
        const char *needs;
    } rules[] = {
        {c.cac != 0, "complex-as-channels spectrograms (cac = true)"},
        {c.nfft == 4096, "nfft = 4096"},
        {c.kernel_size == 8 && c.stride == 4, "encoder kernel 8 with stride 4"},
        {c.audio_channels == 2, "stereo audio"},
        {c.sources == 4, "four sources"},
        {bins_survive, "frequency bins left after every encoder level"},
        {c.context == 1, "context = 1"},
        {c.bottom_channels > 0, "a transformer width (bottom_channels > 0)"},
        {c.t_heads > 0 && c.bottom_channels % std::max(c.t_heads, 1) == 0 &&
             c.bottom_channels / std::max(c.t_heads, 1) == 64,
         "attention heads 64 wide"},
    };
    for (const auto &rule : rules)
        if (!rule.ok) throw_error(DMX_ERR_UNSUPPORTED, std::string("unsupported htdemucs configuration: this backend needs ") +
                                                           rule.needs);
    if (c.segment <= 0.0) throw_error(DMX_ERR_CONFIG, "segment must be positive");
}

// Positional embeddings (host.rs:1078-1122), computed once per shape on the host.
float *pos2d_for(dmx_runner &r, int64_t freqs, int64_t frames) {
    auto key = std::make_pair(freqs, frames);
    auto it = r.pos2d.find(key);
    if (it != r.pos2d.end()) return it->second;
    const int64_t dim = r.tch, half = dim / 2, pairs = half / 2;
    const float max_period = (float)r.cfg.t_max_period;
    const float log_period = std::log(max_period) / (float)half;
    std::vector<float> div(pairs), out(frames * freqs * dim);
    for (int64_t j = 0; j < pairs; ++j) div[j] = std::exp(-(float)(2 * j) * log_period);
    for (int64_t t = 0; t < frames; ++t)
        for (int64_t f = 0; f < freqs; ++f) {
            float *tok = out.data() + (t * freqs + f) * dim;
            for (int64_t j = 0; j < pairs; ++j) {
                float a = (float)t * div[j], b = (float)f * div[j];
                tok[2 * j] = std::sin(a);
                tok[2 * j + 1] = std::cos(a);
                tok[half + 2 * j] = std::sin(b);
                tok[half + 2 * j + 1] = std::cos(b);
            }
        }
    return r.pos2d[key] = upload(r, out);
}

float *pos1d_for(dmx_runner &r, int64_t length) {
    auto it = r.pos1d.find(length);
    if (it != r.pos1d.end()) return it->second;
    const int64_t dim = r.tch, half = dim / 2;
    const float max_period = (float)r.cfg.t_max_period;
    std::vector<float> out(length * dim);
    for (int64_t t = 0; t < length; ++t)
        for (int64_t i = 0; i < half; ++i) {
            float exponent = (float)i / ((float)half - 1.0f);
            float phase = (float)t / std::pow(max_period, exponent);
            out[t * dim + i] = std::cos(phase);
            out[t * dim + half + i] = std::sin(phase);
        }
    return r.pos1d[length] = upload(r, out);
}

// `transition_weight` (crates/demucs-core/src/demucs/pipeline.rs:117-131), power 1.
std::vector<float> transition_weight(int64_t n, double power) {
    std::vector<float> w;
    w.reserve(n);
    int64_t half = n / 2;
    for (int64_t i = 1; i <= half; ++i) w.push_back((float)i);
    for (int64_t i = n - half; i >= 1; --i) w.push_back((float)i);
    float mx = 1.0f;
    for (float v : w) mx = std::max(mx, v);
    for (float &v : w) v = std::pow(v / mx, (float)power);
    return w;
}

// ----- the forward -----

void run_dconv(dmx_runner &r, hipStream_t s, float *x, int B, int C, int F, int T, const LayerW &L) {
    const int rows = B * F;
    if (L.dconv[0].w1_t && L.dconv[1].w1_t && L.dconv[0].hidden == L.dconv[1].hidden) {
        DConvRowLayer rl[2];
        for (int d = 0; d < 2; ++d) {
            const DConvW &D = L.dconv[d];
            rl[d] = {D.w1_t, D.b1, D.n1w, D.n1b, D.w2, D.b2, D.n2w, D.n2b, D.gamma};
        }
        if (dconv_rows(s, x, B, C, F, T, L.dconv[0].hidden, rl)) return;
    }
    // DMX_DCONV_GRAM=0 takes conv2's moments from a conv2 pass instead of
    // the Gram matrix (tuning).
    const char *gram_env = std::getenv("DMX_DCONV_GRAM");
    const bool use_gram = !gram_env || std::atoi(gram_env) != 0;
    for (int d = 0; d < 2; ++d) {
        const DConvW &D = L.dconv[d];
        DBuf h = fbuf(s, dconv_hidden_floats(rows, D.hidden, T));
        DBuf st = dbuf(s, 4 * (int64_t)rows);
        dconv_layer(s, x, B, C, F, T, 1 << d, D.w1, D.w1_gemm, D.w1_t, D.b1, D.hidden, D.n1w, D.n1b, D.w2, D.b2,
                    D.n2w, D.n2b, D.gamma, use_gram ? D.gram : nullptr, h.f(), st.d());
    }
    (void)r;
}

// One `classic_layer_forward` / `cross_layer_forward` (host.rs:1315-1429) on
// token planes, in two halves around the attention core so that the two
// branches' attentions can share one launch.
//
// attention_inputs(): LN1 (and LN2 of the key/value plane for a cross layer)
// and the in-projections, on stream s, into `proj`: a (B, Lq, 3D) q|k|v plane
// for self-attention, or q (B, Lq, D) followed by k|v (B, Lk, 2D) for cross
// attention. Returns the attention problem that reads it.
struct LayerShape {
    int64_t Lq, Lk;  // Lk = Lq for self-attention
    int B;
};
// Whether the layer's attention runs on the three-plane kernel, with the
// in-projection writing K and V as planes.
bool kv_planes(const dmx_runner &r) { return r.planes == 3 && attention_planes_enabled(); }
// The in-projection output for the three-plane attention inside `proj`: q
// (B, Lq, D) fp32, then the K planes [3][B][Lk][D], then the V^T planes
// [3][B * D][ldvt] (KVPlanes).
KVPlanes kv_layout(float *proj, int D, const LayerShape &sh) {
    const int64_t ldvt = kv_ldvt(sh.Lk);
    KVPlanes kv;
    kv.k = reinterpret_cast<unsigned short *>(proj + (int64_t)sh.B * sh.Lq * D);
    kv.ldk = D;
    kv.k_bs = sh.Lk * D;
    kv.k_stride = (int64_t)sh.B * sh.Lk * D;
    kv.vt = kv.k + 3 * kv.k_stride;
    kv.ldvt = ldvt;
    kv.vt_stride = (int64_t)sh.B * D * ldvt;
    return kv;
}
int64_t projection_floats(const dmx_runner &r, const TLayerW &L, const LayerShape &sh) {
    const int D = r.tch;
    if (kv_planes(r)) {
        // q, then 3 K planes and 3 V^T planes of bf16 (half a float each).
        const int64_t halves = 3 * (int64_t)sh.B * sh.Lk * D + 3 * (int64_t)sh.B * D * kv_ldvt(sh.Lk);
        return (int64_t)sh.B * sh.Lq * D + (halves + 1) / 2;
    }
    return L.cross ? sh.B * sh.Lq * D + sh.B * sh.Lk * 2 * D : sh.B * sh.Lq * 3 * D;
}
AttentionArgs attention_inputs(dmx_runner &r, hipStream_t s, const TLayerW &L, const float *xq, const float *xkv,
                               const LayerShape &sh, float *proj, void *att) {
    const int D = r.tch, heads = r.cfg.t_heads, B = sh.B, P = r.planes;
    const int64_t Lq = sh.Lq, Lk = sh.Lk;
    AttentionArgs a{};
    if (kv_planes(r)) {
        // LN1 (LN2 of the key/value plane) as planes, then the in-projection
        // straight into q and the K / V^T planes of the three-plane kernel.
        const KVPlanes kv = kv_layout(proj, D, sh);
        if (sh.Lk % 32 != 0) zero_floats(s, reinterpret_cast<float *>(kv.vt), 3 * kv.vt_stride / 2);
        DBuf nq = obuf(s, B * Lq * D, P);
        const Planes nqp = planes_in(nq, B * Lq * D, P);
        layer_norm_planes(s, xq, (int)(B * Lq), D, L.n1w, L.n1b, nqp);
        if (L.cross) {
            DBuf nk = obuf(s, B * Lk * D, P);
            const Planes nkp = planes_in(nk, B * Lk * D, P);
            layer_norm_planes(s, xkv, (int)(B * Lk), D, L.n2w, L.n2b, nkp);
            linear_planes(s, nqp, D, Lq * D, L.in_wp, L.in_b, B, (int)Lq, D, D, proj, Planes{}, D, Lq * D, TAIL_BIAS,
                          nullptr, nullptr, nullptr);
            linear_qkv_planes(s, nkp, D, Lk * D, L.in_wp.offset((int64_t)D * D), L.in_b + D, B, (int)Lk, D, 2 * D,
                              0, nullptr, kv);
        } else {
            linear_qkv_planes(s, nqp, D, Lq * D, L.in_wp, L.in_b, B, (int)Lq, D, 3 * D, D, proj, kv);
        }
        a = AttentionArgs{proj,  D,     nullptr, D,       nullptr,   D,      nullptr, D,
                          B,     heads, (int)Lq, (int)Lk, D / heads, Lq * D, Lk * D,  Lq * D};
        a.kv = kv;
    } else if (L.cross) {
        float *q = proj, *kv = proj + B * Lq * D;
        if (P) {
            DBuf nq = obuf(s, B * Lq * D, P), nk = obuf(s, B * Lk * D, P);
            const Planes nqp = planes_in(nq, B * Lq * D, P), nkp = planes_in(nk, B * Lk * D, P);
            layer_norm_planes(s, xq, (int)(B * Lq), D, L.n1w, L.n1b, nqp);
            layer_norm_planes(s, xkv, (int)(B * Lk), D, L.n2w, L.n2b, nkp);
            linear_planes(s, nqp, D, Lq * D, L.in_wp, L.in_b, B, (int)Lq, D, D, q, Planes{}, D, Lq * D, TAIL_BIAS,
                          nullptr, nullptr, nullptr);
            linear_planes(s, nkp, D, Lk * D, L.in_wp.offset((int64_t)D * D), L.in_b + D, B, (int)Lk, D, 2 * D, kv,
                          Planes{}, 2 * D, Lk * 2 * D, TAIL_BIAS, nullptr, nullptr, nullptr);
        } else {
            DBuf nq = fbuf(s, B * Lq * D), nk = fbuf(s, B * Lk * D);
            layer_norm_rows(s, xq, (int)(B * Lq), D, L.n1w, L.n1b, nq.f(), nullptr, 0);
            layer_norm_rows(s, xkv, (int)(B * Lk), D, L.n2w, L.n2b, nk.f(), nullptr, 0);
            linear(s, nq.f(), D, Lq * D, L.in_w, L.in_b, B, (int)Lq, D, D, q, D, Lq * D, TAIL_BIAS, nullptr, nullptr,
                   nullptr);
            linear(s, nk.f(), D, Lk * D, L.in_w + (int64_t)D * D, L.in_b + D, B, (int)Lk, D, 2 * D, kv, 2 * D,
                   Lk * 2 * D, TAIL_BIAS, nullptr, nullptr, nullptr);
        }
        a = AttentionArgs{q,     D,     kv,      2 * D,   kv + D,    2 * D,  nullptr,    D,
                          B,     heads, (int)Lq, (int)Lk, D / heads, Lq * D, Lk * 2 * D, Lq * D};
    } else {
        if (P) {
            DBuf nq = obuf(s, B * Lq * D, P);
            const Planes nqp = planes_in(nq, B * Lq * D, P);
            layer_norm_planes(s, xq, (int)(B * Lq), D, L.n1w, L.n1b, nqp);
            linear_planes(s, nqp, D, Lq * D, L.in_wp, L.in_b, B, (int)Lq, D, 3 * D, proj, Planes{}, 3 * D,
                          Lq * 3 * D, TAIL_BIAS, nullptr, nullptr, nullptr);
        } else {
            DBuf nq = fbuf(s, B * Lq * D);
            layer_norm_rows(s, xq, (int)(B * Lq), D, L.n1w, L.n1b, nq.f(), nullptr, 0);
            linear(s, nq.f(), D, Lq * D, L.in_w, L.in_b, B, (int)Lq, D, 3 * D, proj, 3 * D, Lq * 3 * D, TAIL_BIAS,
                   nullptr, nullptr, nullptr);
        }
        a = AttentionArgs{proj, 3 * D, proj + D, 3 * D,    proj + 2 * D, 3 * D,          nullptr,        D,
                          B,    heads, (int)Lq,  (int)Lq,  D / heads,    Lq * 3 * D, Lq * 3 * D, Lq * D};
    }
    // The attention output feeds the out-projection: planes when it reads planes.
    if (P)
        a.out_planes = Planes{static_cast<unsigned short *>(att), plane_stride(B * Lq * D), P};
    else
        a.out = static_cast<float *>(att);
    return a;
}

// attention_outputs(): out-projection + LayerScale residual, LN2/LN3, FFN,
// residual, GroupNorm(1) over the plane, on stream s; writes out (B, Lq, D).
// `att` is what attention_inputs() directed the attention output to.
void attention_outputs(dmx_runner &r, hipStream_t s, const TLayerW &L, const float *xq, const LayerShape &sh,
                       const void *att, const std::string &name, float *out) {
    const int D = r.tch, H = r.hidden, B = sh.B, P = r.planes;
    const int64_t Lq = sh.Lq;
    const float *nw = L.cross ? L.n3w : L.n2w, *nb = L.cross ? L.n3b : L.n2b;
    DBuf x1 = fbuf(s, B * Lq * D);
    DBuf stats = dbuf(s, 2 * B);
    zero_doubles(s, stats.d(), 2 * B);
    if (P) {
        const Planes attp{static_cast<unsigned short *>(const_cast<void *>(att)), plane_stride(B * Lq * D), P};
        linear_planes(s, attp, D, Lq * D, L.out_wp, L.out_b, B, (int)Lq, D, D, x1.f(), Planes{}, D, Lq * D,
                      TAIL_RESIDUAL_SCALE, xq, L.g1, nullptr);
        DBuf n2 = obuf(s, B * Lq * D, P);
        const Planes n2p = planes_in(n2, B * Lq * D, P);
        layer_norm_planes(s, x1.f(), (int)(B * Lq), D, nw, nb, n2p);
        DBuf hid = obuf(s, B * Lq * H, P);
        const Planes hidp = planes_in(hid, B * Lq * H, P);
        linear_planes(s, n2p, D, Lq * D, L.w1p, L.b1, B, (int)Lq, D, H, nullptr, hidp, H, Lq * H, TAIL_BIAS_GELU,
                      nullptr, nullptr, nullptr);
        linear_planes(s, hidp, H, Lq * H, L.w2p, L.b2, B, (int)Lq, H, D, out, Planes{}, D, Lq * D,
                      TAIL_RESIDUAL_SCALE, x1.f(), L.g2, stats.d());
    } else {
        linear(s, static_cast<const float *>(att), D, Lq * D, L.out_w, L.out_b, B, (int)Lq, D, D, x1.f(), D, Lq * D,
               TAIL_RESIDUAL_SCALE, xq, L.g1, nullptr);
        DBuf n2 = fbuf(s, B * Lq * D);
        layer_norm_rows(s, x1.f(), (int)(B * Lq), D, nw, nb, n2.f(), nullptr, 0);
        DBuf hid = fbuf(s, B * Lq * H);
        linear(s, n2.f(), D, Lq * D, L.w1, L.b1, B, (int)Lq, D, H, hid.f(), H, Lq * H, TAIL_BIAS_GELU, nullptr,
               nullptr, nullptr);
        linear(s, hid.f(), H, Lq * H, L.w2, L.b2, B, (int)Lq, H, D, out, D, Lq * D, TAIL_RESIDUAL_SCALE, x1.f(), L.g2,
               stats.d());
    }
    group_norm_tokens_apply(s, out, B, (int)Lq, D, stats.d(), L.now_, L.nob);
    record(r, name, out, {B, Lq, D});
}

// The layers of the cross-transformer (host.rs:895-941) on the token planes
// spec (B, Lf, D) and time (B, Lt, D), which are replaced by the outputs.
#ifndef DMX_ATT_SPLIT
#define DMX_ATT_SPLIT 1
#endif

// Per layer the two branches run concurrently, the waveform branch on the
// side stream; the streams join at layer boundaries, since cross layers read
// the other branch's plane of layer i - 1. (DMX_ATT_SPLIT=0: both attentions
// share one launch on s between a join and a second fork.)
void transformer_layers(dmx_runner &r, hipStream_t s, DBuf &spec, int64_t Lf, DBuf &time, int64_t Lt, int B) {
    const int D = r.tch, heads = r.cfg.t_heads;
    const float scale = 1.0f / std::sqrt((float)(D / heads));
    for (int i = 0; i < r.cfg.t_layers; ++i) {
        std::string n = "crosstransformer.layers." + std::to_string(i);
        std::string nt = "crosstransformer.layers_t." + std::to_string(i);
        const TLayerW &Ls = r.layers[i], &Lt_ = r.layers_t[i];
        const bool cross = Ls.cross;
        const LayerShape shs{Lf, cross ? Lt : Lf, B}, sht{Lt, cross ? Lf : Lt, B};
        // Everything both streams touch comes from s's pool, before the fork.
        DBuf ns = fbuf(s, B * Lf * D), nt_ = fbuf(s, (int64_t)B * Lt * D);
        DBuf ps = fbuf(s, projection_floats(r, Ls, shs)), pt = fbuf(s, projection_floats(r, Lt_, sht));
        DBuf as = obuf(s, B * Lf * D, r.planes), at = obuf(s, (int64_t)B * Lt * D, r.planes);
        Branches br(r, s);
        br.fork();
#if DMX_ATT_SPLIT
        // Within a layer the branches do not depend on each other (a cross
        // layer reads the other branch's plane of layer i - 1, which both
        // streams have at the fork): each branch runs projections, its
        // attention and its output half on its own stream, and the shorter
        // time-branch chain fills the tail of the spectral attention.
        {
            const AttentionArgs pta =
                attention_inputs(r, br.t, Lt_, time.f(), cross ? spec.f() : nullptr, sht, pt.f(), at.p);
            attention_grouped(br.t, &pta, 1, scale);
            attention_outputs(r, br.t, Lt_, time.f(), sht, at.p, nt, nt_.f());
            const AttentionArgs psa =
                attention_inputs(r, s, Ls, spec.f(), cross ? time.f() : nullptr, shs, ps.f(), as.p);
            attention_grouped(s, &psa, 1, scale);
            attention_outputs(r, s, Ls, spec.f(), shs, as.p, n, ns.f());
        }
        br.join();
#else
        AttentionArgs prob[2];
        prob[1] = attention_inputs(r, br.t, Lt_, time.f(), cross ? spec.f() : nullptr, sht, pt.f(), at.p);
        prob[0] = attention_inputs(r, s, Ls, spec.f(), cross ? time.f() : nullptr, shs, ps.f(), as.p);
        br.join();
        attention_grouped(s, prob, 2, scale);
        Branches br2(r, s);
        br2.fork();
        attention_outputs(r, br2.t, Lt_, time.f(), sht, at.p, nt, nt_.f());
        attention_outputs(r, s, Ls, spec.f(), shs, as.p, n, ns.f());
        br2.join();
#endif
        spec = std::move(ns);
        time = std::move(nt_);
        if (r.mark_mid == 30 + i) DMX_HIP(hipEventRecord(r.ev_mid, s));
    }
}

// `transformer_forward` (host.rs:830-946): x (B, D, F, T), xt (B, D, Lt) channel-major.
void transformer(dmx_runner &r, hipStream_t s, const float *x, const float *xt, int B, int F, int T, int Lt,
                 float *x_out, float *xt_out) {
    const int D = r.tch;
    const int64_t Lf = (int64_t)F * T;
    const float wpe = (float)r.cfg.t_weight_pos_embed;
    DBuf spec = fbuf(s, B * Lf * D), time = fbuf(s, (int64_t)B * Lt * D);
    channels_to_tokens_ln(s, x, B, D, F, T, dev(r, "crosstransformer.norm_in.weight"),
                          dev(r, "crosstransformer.norm_in.bias"), pos2d_for(r, F, T), wpe, spec.f());
    channels_to_tokens_ln(s, xt, B, D, 1, Lt, dev(r, "crosstransformer.norm_in_t.weight"),
                          dev(r, "crosstransformer.norm_in_t.bias"), pos1d_for(r, Lt), wpe, time.f());
    record(r, "crosstransformer.in#0", spec.f(), {B, Lf, D});
    record(r, "crosstransformer.in#1", time.f(), {B, Lt, D});
    transformer_layers(r, s, spec, Lf, time, Lt, B);
    // The channel downsamplers read the token planes directly.
    tokens_to_channels(s, spec.f(), B, F, T, D, dev(r, "channel_downsampler.weight"), dev(r, "channel_downsampler.bias"),
                       r.pre_channels, x_out);
    tokens_to_channels(s, time.f(), B, 1, Lt, D, dev(r, "channel_downsampler_t.weight"),
                       dev(r, "channel_downsampler_t.bias"), r.pre_channels, xt_out);
}

// Stack-only entry point: same prologue/layers, outputs rearranged back to
// (B, D, F, T) / (B, D, Lt) without the channel mixers.
// The runner's precision as the MFMA input precision of what it launches.
MfmaPrecision mfma_of(const dmx_runner &r) { return mfma_of_precision(r.precision); }

void transformer_only(dmx_runner &r, hipStream_t s, const float *x, const float *xt, int B, int F, int T, int Lt,
                      float *x_out, float *xt_out) {
    MfmaPrecisionScope prec(mfma_of(r));
    const int D = r.tch;
    const int64_t Lf = (int64_t)F * T;
    const float wpe = (float)r.cfg.t_weight_pos_embed;
    DBuf spec = fbuf(s, B * Lf * D), time = fbuf(s, (int64_t)B * Lt * D);
    channels_to_tokens_ln(s, x, B, D, F, T, dev(r, "crosstransformer.norm_in.weight"),
                          dev(r, "crosstransformer.norm_in.bias"), pos2d_for(r, F, T), wpe, spec.f());
    channels_to_tokens_ln(s, xt, B, D, 1, Lt, dev(r, "crosstransformer.norm_in_t.weight"),
                          dev(r, "crosstransformer.norm_in_t.bias"), pos1d_for(r, Lt), wpe, time.f());
    transformer_layers(r, s, spec, Lf, time, Lt, B);
    // The rearrange back to (B, D, F, T) reuses the token-gather GEMM with an
    // identity matrix (exact: every output is one product by 1.0 plus zeros).
    if (!r.eye) {
        std::vector<float> eye((size_t)D * D + D, 0.0f);
        for (int i = 0; i < D; ++i) eye[(size_t)i * D + i] = 1.0f;
        r.eye = upload(r, eye);
    }
    tokens_to_channels(s, spec.f(), B, F, T, D, r.eye, r.eye + (size_t)D * D, D, x_out);
    tokens_to_channels(s, time.f(), B, 1, Lt, D, r.eye, r.eye + (size_t)D * D, D, xt_out);
}

// `Htdemucs::forward` on device: mix (B, 2, L) with L == training_length -> stems (B, S, 2, L).
void forward_full(dmx_runner &r, hipStream_t s, const float *mix, int B, float *stems) {
    MfmaPrecisionScope prec(mfma_of(r));
    const dmx_config &c = r.cfg;
    const int L = (int)r.training_length, nfft = c.nfft, hop = r.hop, le = (int)ceil_div(L, hop), bins = nfft / 2;
    DBuf frames = fbuf(s, (int64_t)B * 2 * le * bins * 2);
    DBuf xspec = fbuf(s, (int64_t)B * 4 * bins * le);
    DBuf xwave = fbuf(s, (int64_t)B * 2 * L);
    DBuf norms = fbuf(s, 4 * (int64_t)B);
    DBuf nstats = dbuf(s, 4 * (int64_t)B);
    spec_and_normalise(s, mix, B, L, nfft, frames.f(), xspec.f(), xwave.f(), norms.f(), nstats.d(), r.twiddles);
    frames.release();
    record(r, "x_normalized", xspec.f(), {B, 4, bins, le});
    record(r, "xt_normalized", xwave.f(), {B, 2, L});

    const int depth = c.depth;
    std::vector<DBuf> saved, saved_t;
    std::vector<int> lengths_t;
    // The waveform encoder's outputs are also the waveform decoder's skips:
    // s's pool, taken before the fork, released after the decoder's join.
    int tlen = L;
    for (int i = 0; i < depth; ++i) {
        lengths_t.push_back(tlen);
        const int padded = tlen % 4 ? tlen + (4 - tlen % 4) : tlen;
        tlen = (padded + 4 - 8) / 4 + 1;
        saved_t.push_back(fbuf(s, (int64_t)B * r.tenc[i].cout * tlen));
    }
    Branches enc(r, s);
    enc.fork();
    // Layer i of both encoders is enqueued together (the waveform layer on
    // the side stream), so neither stream waits for the host to enqueue the
    // other branch's whole encoder.
    const float *xt_in = xwave.f();
    int tcin = 2;
    // Each encoder layer reads the previous layer's output, which is also the
    // skip connection kept in saved.
    const float *x_in = xspec.f();
    int cin = 4, F = bins;
    for (int i = 0; i < depth; ++i) {
        {
            // Waveform encoder (host.rs:625-678).
            const hipStream_t t = enc.t;
            const LayerW &TL = r.tenc[i];
            const int len = lengths_t[i];
            const int padded = len % 4 ? len + (4 - len % 4) : len;
            const int tout = (padded + 4 - 8) / 4 + 1;
            DBuf y = fbuf(t, (int64_t)B * TL.cout * tout);
            conv1d_right_padded(t, xt_in, B, tcin, len, padded, TL.conv_w, TL.conv_b, TL.cout, 8, 4, 2, y.f(),
                                ACT_GELU);
            run_dconv(r, t, y.f(), B, TL.cout, 1, tout, TL);
            conv2d_glu(t, y.f(), nullptr, B, TL.cout, 1, tout, TL.rw, TL.rb, TL.cout, 1, 1, 0, 0, saved_t[i].f(),
                       nullptr, 0.f);
            tcin = TL.cout;
            record(r, "tencoder." + std::to_string(i), saved_t[i].f(), {B, tcin, tout});
            xt_in = saved_t[i].f();
        }
        // Frequency encoder (host.rs:577-622).
        const LayerW &FL = r.enc[i];
        int fout = (F + 4 - 8) / 4 + 1;
        DBuf yf = fbuf(s, (int64_t)B * FL.cout * fout * le);
        conv2d(s, x_in, nullptr, B, cin, F, le, FL.conv_w, FL.conv_b, FL.cout, 8, 1, 4, 1, 2, 0, 1, 1, yf.f(), ACT_GELU);
        run_dconv(r, s, yf.f(), B, FL.cout, fout, le, FL);
        DBuf x_next = fbuf(s, (int64_t)B * FL.cout * fout * le);
        const bool emb = i == 0 && c.freq_emb > 0.0;
        if (emb) DMX_REQUIRE(fout == r.freq_emb_rows && FL.cout == c.channels, "frequency embedding shape mismatch");
        conv2d_glu(s, yf.f(), nullptr, B, FL.cout, fout, le, FL.rw, FL.rb, FL.cout, 1, 1, 0, 0, x_next.f(),
                   emb ? r.freq_emb : nullptr, (float)c.freq_emb);
        cin = FL.cout;
        F = fout;
        if (wants(r, "encoder." + std::to_string(i)) && !emb)
            record(r, "encoder." + std::to_string(i), x_next.f(), {B, cin, F, le});
        if (emb) record(r, "encoder.0.post_emb", x_next.f(), {B, cin, F, le});
        x_in = x_next.f();
        saved.push_back(std::move(x_next));
        if (r.mark_mid == 10 + i) DMX_HIP(hipEventRecord(r.ev_mid, s));
    }
    enc.join();
    xspec.release();
    xwave.release();
    const float *xin = saved.back().f();
    const float *xtin = saved_t.back().f();
    // Channel upsamplers (host.rs:320-339) then the transformer.
    const int D = r.tch, P = r.pre_channels;
    DBuf up = fbuf(s, (int64_t)B * D * F * le), upt = fbuf(s, (int64_t)B * D * tlen);
    pointwise(s, dev(r, "channel_upsampler.weight"), dev(r, "channel_upsampler.bias"), xin, B, D, P, F * le, up.f(),
              ACT_NONE);
    pointwise(s, dev(r, "channel_upsampler_t.weight"), dev(r, "channel_upsampler_t.bias"), xtin, B, D, P, tlen,
              upt.f(), ACT_NONE);
    record(r, "channel_upsampler", up.f(), {B, D, (int64_t)F * le});
    record(r, "channel_upsampler_t", upt.f(), {B, D, tlen});
    DBuf xd = fbuf(s, (int64_t)B * P * F * le), xtd = fbuf(s, (int64_t)B * P * tlen);
    if (r.mark_mid == 1) DMX_HIP(hipEventRecord(r.ev_mid, s));
    transformer(r, s, up.f(), upt.f(), B, F, le, tlen, xd.f(), xtd.f());
    if (r.mark_mid == 2) DMX_HIP(hipEventRecord(r.ev_mid, s));
    up.release();
    upt.release();
    record(r, "channel_downsampler", xd.f(), {B, P, (int64_t)F * le});
    record(r, "channel_downsampler_t", xtd.f(), {B, P, tlen});

    // Decoders: the waveform branch on the side stream again. Its last
    // output feeds the final sum on s, so it comes from s's pool.
    DBuf xt_out = fbuf(s, (int64_t)B * c.sources * 2 * L);
    Branches dec(r, s);
    dec.fork();
    // Layer i of both decoders is enqueued together, the waveform layer on
    // the side stream.
    const float *xt_in2 = xtd.f();
    DBuf cur;  // the waveform decoder's previous output (side-stream pool)
    int tc = P;
    DBuf x = std::move(xd);
    cin = P;
    for (int i = 0; i < depth; ++i) {
        const bool last = i == depth - 1;
        {
            // Waveform decoder (host.rs:763-827).
            const hipStream_t t = dec.t;
            const LayerW &TL = r.tdec[i];
            const float *skip_t = saved_t[depth - 1 - i].f();
            const int length_t = lengths_t[depth - 1 - i];
            DBuf gt = fbuf(t, (int64_t)B * tc * tlen);
            conv2d_glu(t, xt_in2, skip_t, B, tc, 1, tlen, TL.rw, TL.rb, tc, 1, 3, 0, 1, gt.f(), nullptr, 0.f);
            run_dconv(r, t, gt.f(), B, tc, 1, tlen, TL);
            record(r, "tdecoder." + std::to_string(i) + "#1", gt.f(), {B, tc, tlen});
            DBuf zt = last ? DBuf() : fbuf(t, (int64_t)B * TL.cout * length_t);
            float *zt_p = last ? xt_out.f() : zt.f();
            conv_transpose_axis(t, gt.f(), B, tc, tlen, 1, TL.conv_w, TL.conv_b, TL.cout, 8, 4, 2, length_t, zt_p,
                                last ? ACT_NONE : ACT_GELU);
            record(r, "tdecoder." + std::to_string(i) + "#0", zt_p, {B, TL.cout, length_t});
            cur = std::move(zt);
            xt_in2 = zt_p;
            tc = TL.cout;
            tlen = length_t;
        }
        // Frequency decoder (host.rs:682-759).
        const LayerW &FL = r.dec[i];
        DBuf skip = std::move(saved.back());
        saved.pop_back();
        DBuf g = fbuf(s, (int64_t)B * cin * F * le);
        if (FL.rw_wino && winograd_applies(cin, cin, F, le)) {
            DBuf ws = fbuf(s, winograd_scratch_floats(B, cin, cin, F, le));
            conv3x3_glu_winograd(s, x.f(), skip.f(), B, cin, cin, F, le, FL.rw_wino, FL.rb, g.f(), ws.f());
        } else {
            conv2d_glu(s, x.f(), skip.f(), B, cin, F, le, FL.rw, FL.rb, cin, 3, 3, 1, 1, g.f(), nullptr, 0.f);
        }
        skip.release();
        run_dconv(r, s, g.f(), B, cin, F, le, FL);
        record(r, "decoder." + std::to_string(i) + "#1", g.f(), {B, cin, F, le});
        int fout = 4 * F;
        DBuf z = fbuf(s, (int64_t)B * FL.cout * fout * le);
        conv_transpose_axis(s, g.f(), B, cin, F, le, FL.conv_w, FL.conv_b, FL.cout, 8, 4, 2, fout, z.f(),
                            last ? ACT_NONE : ACT_GELU);
        record(r, "decoder." + std::to_string(i) + "#0", z.f(), {B, FL.cout, fout, le});
        if (r.mark_mid == 20 + i) DMX_HIP(hipEventRecord(r.ev_mid, s));
        x = std::move(z);
        cin = FL.cout;
        F = fout;
    }
    DMX_REQUIRE(tc == c.sources * 2 && tlen == L, "waveform decoder output shape is wrong");
    dec.join();
    saved_t.clear();
    xtd.release();
    DMX_REQUIRE(cin == c.sources * 4, "decoder output shapes are wrong");
    const DBuf &xt = xt_out;
    const int S = c.sources, rows = B * S * 2;
    DBuf scratch = fbuf(s, (int64_t)rows * le * nfft + (int64_t)rows * le * bins * 2);
    ispec_and_sum(s, x.f(), xt.f(), B, S, L, nfft, le, norms.f(), scratch.f(), stems, r.twiddles);
    record(r, "model_out", stems, {B, S, 2, L});
}

// Forward with any length <= training_length: zero pad in, crop out.
void forward_device(dmx_runner &r, hipStream_t s, const float *mix, int64_t B, int64_t channels, int64_t length,
                    float *stems) {
    if (channels != r.cfg.audio_channels)
        throw_error(DMX_ERR_SHAPE, "expected " + std::to_string(r.cfg.audio_channels) + " audio channels, got " +
                                       std::to_string(channels));
    const int64_t L = r.training_length;
    if (length > L)
        throw_error(DMX_ERR_SHAPE, "input is " + std::to_string(length) + " samples but the model segment is " +
                                       std::to_string(L) + "; chunk the audio before calling forward");
    if (B <= 0 || length <= 0) throw_error(DMX_ERR_SHAPE, "empty input");
    const int S = r.cfg.sources;
    if (length == L) {
        forward_full(r, s, mix, (int)B, stems);
        return;
    }
    DBuf padded = fbuf(s, B * channels * L), full = fbuf(s, B * S * 2 * L);
    copy_rows(s, mix, B * channels, length, length, padded.f(), L);
    forward_full(r, s, padded.f(), (int)B, full.f());
    copy_rows(s, full.f(), B * S * 2, L, length, stems, length);
}

// ----- weights -----

// The transformer linears' weights as bf16 planes, split once on the device
// (one block for all of them).
void split_linear_weights(dmx_runner &r) {
    const int P = r.planes, D = r.tch, H = r.hidden;
    const int64_t sizes[4] = {3LL * D * D, (int64_t)D * D, (int64_t)H * D, (int64_t)D * H};
    int64_t per_layer = 0;
    for (int64_t n : sizes) per_layer += plane_stride(n) * P;
    const size_t n_layers = r.layers.size() + r.layers_t.size();
    void *mem = nullptr;
    DMX_HIP(hipMalloc(&mem, std::max<size_t>(n_layers * per_layer * sizeof(unsigned short), 16)));
    r.owned.push_back(mem);
    unsigned short *at = static_cast<unsigned short *>(mem);
    auto take = [&](const float *w, int64_t n) {
        const Planes p{at, plane_stride(n), P};
        split_to_planes(r.stream, w, n, p);
        at += plane_stride(n) * P;
        return p;
    };
    for (auto *v : {&r.layers, &r.layers_t})
        for (TLayerW &L : *v) {
            L.in_wp = take(L.in_w, sizes[0]);
            L.out_wp = take(L.out_w, sizes[1]);
            L.w1p = take(L.w1, sizes[2]);
            L.w2p = take(L.w2, sizes[3]);
        }
}

void load_weights(dmx_runner &r, const dmx_tensor *weights, size_t n) {
    const dmx_config &c = r.cfg;
    // Expected shapes (crates/demucs-core/src/demucs/weights.rs:224-578, config.rs:325-444).
    std::map<std::string, std::vector<int64_t>> expect;
    std::map<std::string, const dmx_tensor *> given;
    for (size_t i = 0; i < n; ++i) {
        if (!weights[i].name || !weights[i].data) throw_error(DMX_ERR_ARGUMENT, "weight entry without name or data");
        given[weights[i].name] = &weights[i];
    }
    const int depth = c.depth, hidden_div = 8;
    int chin = c.audio_channels, chin_z = chin * 2, chout = c.channels, chout_z = c.channels, freqs = c.nfft / 2;
    struct Spec {
        int chin, chout;
    };
    std::vector<Spec> dspec, tdspec;
    auto dconv_shapes = [&](const std::string &p, int ch) {
        int hid = ch / hidden_div;
        for (int d = 0; d < 2; ++d) {
            std::string at = p + ".layers." + std::to_string(d);
            expect[at + ".0.weight"] = {hid, ch, 3};
            expect[at + ".0.bias"] = {hid};
            expect[at + ".1.weight"] = {hid};
            expect[at + ".1.bias"] = {hid};
            expect[at + ".3.weight"] = {2 * ch, hid, 1};
            expect[at + ".3.bias"] = {2 * ch};
            expect[at + ".4.weight"] = {2 * ch};
            expect[at + ".4.bias"] = {2 * ch};
            expect[at + ".6.scale"] = {ch};
        }
    };
    for (int i = 0; i < depth; ++i) {
        std::string e = "encoder." + std::to_string(i), te = "tencoder." + std::to_string(i);
        expect[e + ".conv.weight"] = {chout_z, chin_z, 8, 1};
        expect[e + ".conv.bias"] = {chout_z};
        expect[e + ".rewrite.weight"] = {2 * chout_z, chout_z, 1, 1};
        expect[e + ".rewrite.bias"] = {2 * chout_z};
        dconv_shapes(e + ".dconv", chout_z);
        expect[te + ".conv.weight"] = {chout, chin, 8};
        expect[te + ".conv.bias"] = {chout};
        expect[te + ".rewrite.weight"] = {2 * chout, chout, 1};
        expect[te + ".rewrite.bias"] = {2 * chout};
        dconv_shapes(te + ".dconv", chout);
        if (i == 0) {
            chin = c.audio_channels * c.sources;
            chin_z = chin * 2;
        }
        dspec.push_back({chout_z, chin_z});
        tdspec.push_back({chout, chin});
        if (i == 0) r.freq_emb_rows = freqs / c.stride;
        chin = chout;
        chin_z = chout_z;
        chout *= c.growth;
        chout_z *= c.growth;
        freqs /= c.stride;
    }
    for (int i = 0; i < depth; ++i) {
        std::string d = "decoder." + std::to_string(i), td = "tdecoder." + std::to_string(i);
        expect[d + ".conv_tr.weight"] = {dspec[i].chin, dspec[i].chout, 8, 1};
        expect[d + ".conv_tr.bias"] = {dspec[i].chout};
        expect[d + ".rewrite.weight"] = {2 * dspec[i].chin, dspec[i].chin, 3, 3};
        expect[d + ".rewrite.bias"] = {2 * dspec[i].chin};
        dconv_shapes(d + ".dconv", dspec[i].chin);
        expect[td + ".conv_tr.weight"] = {tdspec[i].chin, tdspec[i].chout, 8};
        expect[td + ".conv_tr.bias"] = {tdspec[i].chout};
        expect[td + ".rewrite.weight"] = {2 * tdspec[i].chin, tdspec[i].chin, 3};
        expect[td + ".rewrite.bias"] = {2 * tdspec[i].chin};
        dconv_shapes(td + ".dconv", tdspec[i].chin);
    }
    r.pre_channels = chin_z;
    r.tch = c.bottom_channels;
    r.hidden = (int)((double)r.tch * c.t_hidden_scale);
    const int D = r.tch, P = r.pre_channels, H = r.hidden;
    expect["freq_emb.embedding.weight"] = {r.freq_emb_rows, c.channels};
    expect["channel_upsampler.weight"] = {D, P, 1};
    expect["channel_upsampler.bias"] = {D};
    expect["channel_upsampler_t.weight"] = {D, P, 1};
    expect["channel_upsampler_t.bias"] = {D};
    expect["channel_downsampler.weight"] = {P, D, 1};
    expect["channel_downsampler.bias"] = {P};
    expect["channel_downsampler_t.weight"] = {P, D, 1};
    expect["channel_downsampler_t.bias"] = {P};
    for (const char *nm : {"crosstransformer.norm_in", "crosstransformer.norm_in_t"}) {
        expect[std::string(nm) + ".weight"] = {D};
        expect[std::string(nm) + ".bias"] = {D};
    }
    for (int i = 0; i < c.t_layers; ++i)
        for (const char *branch : {"crosstransformer.layers.", "crosstransformer.layers_t."}) {
            std::string p = branch + std::to_string(i);
            bool cross = i % 2 == 1;
            std::string a = p + (cross ? ".cross_attn" : ".self_attn");
            expect[a + ".in_proj_weight"] = {3 * D, D};
            expect[a + ".in_proj_bias"] = {3 * D};
            expect[a + ".out_proj.weight"] = {D, D};
            expect[a + ".out_proj.bias"] = {D};
            expect[p + ".linear1.weight"] = {H, D};
            expect[p + ".linear1.bias"] = {H};
            expect[p + ".linear2.weight"] = {D, H};
            expect[p + ".linear2.bias"] = {D};
            std::vector<std::string> norms = {".norm1", ".norm2", ".norm_out"};
            if (cross) norms.push_back(".norm3");
            for (auto &nm : norms) {
                expect[p + nm + ".weight"] = {D};
                expect[p + nm + ".bias"] = {D};
            }
            expect[p + ".gamma_1.scale"] = {D};
            expect[p + ".gamma_2.scale"] = {D};
        }
    // Check, then upload every expected tensor into one block.
    size_t total = 0;
    for (auto &kv : expect) {
        auto it = given.find(kv.first);
        if (it == given.end()) throw_error(DMX_ERR_MISSING_WEIGHT, "weight `" + kv.first + "` not found in checkpoint");
        const dmx_tensor *t = it->second;
        std::vector<int64_t> shape(t->shape, t->shape + std::max(0, std::min(4, (int)t->ndim)));
        if ((int)t->ndim != (int)kv.second.size() || shape != kv.second) {
            std::string f, e;
            for (auto v : shape) f += std::to_string(v) + ",";
            for (auto v : kv.second) e += std::to_string(v) + ",";
            throw_error(DMX_ERR_WEIGHT_SHAPE, "weight `" + kv.first + "` shape mismatch: checkpoint [" + f +
                                                  "], model expects [" + e + "]");
        }
        int64_t count = 1;
        for (auto v : kv.second) count *= v;
        total += ((size_t)count + 63) / 64 * 64;
    }
    DMX_HIP(hipMalloc(&r.weight_mem, total * sizeof(float)));
    float *base = static_cast<float *>(r.weight_mem);
    size_t off = 0;
    for (auto &kv : expect) {
        const dmx_tensor *t = given[kv.first];
        int64_t count = 1;
        for (auto v : kv.second) count *= v;
        DMX_HIP(hipMemcpy(base + off, t->data, (size_t)count * sizeof(float), hipMemcpyHostToDevice));
        r.w[kv.first] = base + off;
        off += ((size_t)count + 63) / 64 * 64;
    }
    // Derived forms: convT phase packing, scaled frequency embedding.
    auto packed_convt = [&](const std::string &name, int ic, int oc) {
        const dmx_tensor *t = given[name];
        std::vector<float> p((size_t)4 * oc * ic * 2);
        pack_conv_transpose(t->data, ic, oc, 8, 4, p.data());
        return upload(r, p);
    };
    {
        const dmx_tensor *t = given["freq_emb.embedding.weight"];
        std::vector<float> e((size_t)t->shape[0] * t->shape[1]);
        for (size_t i = 0; i < e.size(); ++i) e[i] = t->data[i] * (float)c.emb_scale;
        r.freq_emb = upload(r, e);
    }
    // Conv weights in GEMM order (tap-major where conv_tap_major holds).
    auto gemm_order = [&](const std::string &name, int oc, int ic, int kh, int kw) -> const float * {
        if (!conv_tap_major(ic, kh, kw)) return dev(r, name);
        std::vector<float> g((size_t)oc * ic * kh * kw);
        conv_gemm_weights(given[name]->data, oc, ic, kh, kw, g.data());
        return upload(r, g);
    };
    auto fill_dconv = [&](LayerW &L, const std::string &p, int ch) {
        for (int d = 0; d < 2; ++d) {
            std::string at = p + ".layers." + std::to_string(d);
            const int hid = ch / hidden_div;
            const float *w1_t = nullptr;
            if (dconv_narrow_applies(ch, hid)) {
                std::vector<float> t((size_t)ch * 3 * hid);
                dconv_w1_transposed(given[at + ".0.weight"]->data, ch, hid, t.data());
                w1_t = upload(r, t);
            }
            double *gram = nullptr;
            DMX_HIP(hipMalloc((void **)&gram, (size_t)dconv_gram_doubles(hid) * sizeof(double)));
            r.owned.push_back(gram);
            dconv_gram_weights(r.stream, dev(r, at + ".3.weight"), dev(r, at + ".3.bias"), ch, hid, gram);
            L.dconv[d] = {dev(r, at + ".0.weight"), dev(r, at + ".0.bias"), dev(r, at + ".1.weight"),
                          dev(r, at + ".1.bias"),   dev(r, at + ".3.weight"), dev(r, at + ".3.bias"),
                          dev(r, at + ".4.weight"), dev(r, at + ".4.bias"), dev(r, at + ".6.scale"),
                          hid,                      gemm_order(at + ".0.weight", hid, ch, 1, 3),
                          w1_t,                     gram};
        }
    };
    chin = c.audio_channels;
    chin_z = chin * 2;
    chout = c.channels;
    chout_z = c.channels;
    for (int i = 0; i < depth; ++i) {
        std::string e = "encoder." + std::to_string(i), te = "tencoder." + std::to_string(i);
        LayerW L;
        L.conv_w = gemm_order(e + ".conv.weight", chout_z, chin_z, 8, 1);
        L.conv_b = dev(r, e + ".conv.bias");
        L.rw = dev(r, e + ".rewrite.weight");
        L.rb = dev(r, e + ".rewrite.bias");
        L.cin = chin_z;
        L.cout = chout_z;
        fill_dconv(L, e + ".dconv", chout_z);
        r.enc.push_back(L);
        LayerW T;
        T.conv_w = gemm_order(te + ".conv.weight", chout, chin, 1, 8);
        T.conv_b = dev(r, te + ".conv.bias");
        T.rw = dev(r, te + ".rewrite.weight");
        T.rb = dev(r, te + ".rewrite.bias");
        T.cin = chin;
        T.cout = chout;
        fill_dconv(T, te + ".dconv", chout);
        r.tenc.push_back(T);
        chin = chout;
        chin_z = chout_z;
        chout *= c.growth;
        chout_z *= c.growth;
    }
    for (int i = depth - 1; i >= 0; --i) {
        std::string d = "decoder." + std::to_string(i), td = "tdecoder." + std::to_string(i);
        LayerW L;
        L.cin = dspec[i].chin;
        L.cout = dspec[i].chout;
        L.conv_w = packed_convt(d + ".conv_tr.weight", L.cin, L.cout);
        L.conv_b = dev(r, d + ".conv_tr.bias");
        L.rw = gemm_order(d + ".rewrite.weight", 2 * L.cin, L.cin, 3, 3);
        L.rb = dev(r, d + ".rewrite.bias");
        if (winograd_tile(L.cin, L.cin)) {
            std::vector<float> u((size_t)winograd_weight_floats(L.cin, L.cin));
            winograd_weights(given[d + ".rewrite.weight"]->data, 2 * L.cin, L.cin, u.data());
            L.rw_wino = upload(r, u);
        }
        fill_dconv(L, d + ".dconv", L.cin);
        r.dec.push_back(L);
        LayerW T;
        T.cin = tdspec[i].chin;
        T.cout = tdspec[i].chout;
        T.conv_w = packed_convt(td + ".conv_tr.weight", T.cin, T.cout);
        T.conv_b = dev(r, td + ".conv_tr.bias");
        T.rw = gemm_order(td + ".rewrite.weight", 2 * T.cin, T.cin, 1, 3);
        T.rb = dev(r, td + ".rewrite.bias");
        fill_dconv(T, td + ".dconv", T.cin);
        r.tdec.push_back(T);
    }
    for (int i = 0; i < c.t_layers; ++i)
        for (int branch = 0; branch < 2; ++branch) {
            std::string p = std::string(branch ? "crosstransformer.layers_t." : "crosstransformer.layers.") +
                            std::to_string(i);
            TLayerW L{};
            L.cross = i % 2 == 1;
            std::string a = p + (L.cross ? ".cross_attn" : ".self_attn");
            L.in_w = dev(r, a + ".in_proj_weight");
            L.in_b = dev(r, a + ".in_proj_bias");
            L.out_w = dev(r, a + ".out_proj.weight");
            L.out_b = dev(r, a + ".out_proj.bias");
            L.w1 = dev(r, p + ".linear1.weight");
            L.b1 = dev(r, p + ".linear1.bias");
            L.w2 = dev(r, p + ".linear2.weight");
            L.b2 = dev(r, p + ".linear2.bias");
            L.n1w = dev(r, p + ".norm1.weight");
            L.n1b = dev(r, p + ".norm1.bias");
            L.n2w = dev(r, p + ".norm2.weight");
            L.n2b = dev(r, p + ".norm2.bias");
            if (L.cross) {
                L.n3w = dev(r, p + ".norm3.weight");
                L.n3b = dev(r, p + ".norm3.bias");
            }
            L.now_ = dev(r, p + ".norm_out.weight");
            L.nob = dev(r, p + ".norm_out.bias");
            L.g1 = dev(r, p + ".gamma_1.scale");
            L.g2 = dev(r, p + ".gamma_2.scale");
            (branch ? r.layers_t : r.layers).push_back(L);
        }
    // The plane path covers the model's shapes (rows of 512, K a multiple of 64).
    if (r.tch != 512 || r.hidden % 64 != 0) r.planes = 0;
    if (r.planes) split_linear_weights(r);
    std::vector<float> tw((size_t)c.nfft / 2 * 2 + c.nfft);
    make_twiddles(c.nfft, tw.data());
    r.twiddles = upload(r, tw);
}

void set_device(const dmx_runner *r) { DMX_HIP(hipSetDevice(r->device)); }

// ----- separation (chunk loop on device) -----

struct ShiftRng {
    uint64_t s;
    explicit ShiftRng(uint64_t seed) : s(seed * 6364136223846793005ULL + 1ULL) {}
    int64_t randint(int64_t max) {
        s = s * 6364136223846793005ULL + 1442695040888963407ULL;
        return (int64_t)((s >> 33) % (uint64_t)(max + 1));
    }
};

float *ola_weight_for(dmx_runner &r, int64_t seg, double power) {
    auto key = std::make_pair(seg, power);
    auto it = r.ola_weights.find(key);
    if (it != r.ola_weights.end()) return it->second;
    float *p = upload(r, transition_weight(seg, power));
    r.ola_weights[key] = p;
    return p;
}

// The runner's i-th group-mark event, made on first use.
hipEvent_t mark_event(dmx_runner &r, size_t i) {
    while (r.marks.size() <= i) {
        hipEvent_t e = nullptr;
        DMX_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
        r.marks.push_back(e);
    }
    return r.marks[i];
}

// The runner's i-th readback event, made on first use.
hipEvent_t xfer_event(dmx_runner &r, size_t i) {
    while (r.xfer.size() <= i) {
        hipEvent_t e = nullptr;
        DMX_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
        r.xfer.push_back(e);
    }
    return r.xfer[i];
}

// Largest pinned staging (mix + stems) dmx_separate keeps per runner:
// DMX_PINNED_MAX_MB (read per call), default 1024, about six minutes of four
// stereo stems. Larger calls go through the runner's 24 MB ring instead and
// read the stems back after the last group.
size_t pinned_limit() {
    const char *v = std::getenv("DMX_PINNED_MAX_MB");
    long mb = v ? std::atol(v) : 1024;
    return (size_t)std::max(0L, mb) << 20;
}

// What a caller of separate_device can wait for: `ev` is recorded on the
// runner's main stream after a chunk group's overlap-add; by then `done`
// chunk forwards have finished and, in the last pass, output samples
// [lo, hi) of every wanted row are final in `stems`.
struct GroupMark {
    hipEvent_t ev;
    size_t done;
    int64_t lo, hi;
};

// The chunk loop on the device; enqueues everything and returns at once.
// `marks` receives one entry per chunk group, `total` the progress total.
// `on_final(lo, hi)` (optional) is called while the work is enqueued, right
// after output samples [lo, hi) are finished on the main stream, so the
// caller can queue their readback there in order. `stagger` is the point of
// a lane-0 group's forward where the next lane-1 group starts (see below).
void separate_device(dmx_runner *const *nets, const float *bag_weights, int n_nets, const uint8_t *wanted,
                     const float *mix, int64_t samples, int sample_rate, const dmx_separate_options &o, float *stems,
                     std::vector<GroupMark> &marks, size_t &total, int stagger_default = 0,
                     const std::function<void(int64_t, int64_t)> &on_final = nullptr) {
    if (n_nets < 1 || !nets || !nets[0]) throw_error(DMX_ERR_ARGUMENT, "no network");
    dmx_runner &r0 = *nets[0];
    for (int i = 0; i < n_nets; ++i) {
        if (!nets[i]) throw_error(DMX_ERR_ARGUMENT, "null network in the bag");
        if (nets[i]->device != r0.device) throw_error(DMX_ERR_ARGUMENT, "bag networks must share one device");
        if (nets[i]->cfg.sources != r0.cfg.sources || nets[i]->cfg.samplerate != r0.cfg.samplerate)
            throw_error(DMX_ERR_CONFIG, "bag networks disagree on sources or sample rate");
    }
    if (sample_rate != r0.cfg.samplerate)
        throw_error(DMX_ERR_SHAPE, "audio is at " + std::to_string(sample_rate) + " Hz but the model wants " +
                                       std::to_string(r0.cfg.samplerate) + " Hz");
    if (samples <= 0) throw_error(DMX_ERR_SHAPE, "empty mix");
    const int S = r0.cfg.sources, rows = S * 2;
    hipStream_t s = r0.stream;
    const double seg_s = o.segment > 0 ? o.segment : r0.cfg.segment;
    const int64_t seg = (int64_t)((double)r0.cfg.samplerate * seg_s);
    for (int i = 0; i < n_nets; ++i)
        if (seg > nets[i]->training_length) throw_error(DMX_ERR_SHAPE, "segment longer than the model's");
    const int64_t stride = (int64_t)((1.0 - o.overlap) * (double)seg);
    if (stride <= 0) throw_error(DMX_ERR_SHAPE, "overlap leaves no stride");
    const int group = std::max(1, std::min(o.batch_chunks, 64));
    std::vector<uint8_t> requested(S, 1);
    if (wanted)
        for (int i = 0; i < S; ++i) requested[i] = wanted[i] != 0;
    const bool bag = bag_weights != nullptr;
    std::vector<int> active;
    for (int n = 0; n < n_nets; ++n) {
        if (!bag) {
            if (n == 0) active.push_back(0);
            continue;
        }
        bool needed = false;
        for (int i = 0; i < S; ++i) needed |= bag_weights[n * S + i] != 0.0f && requested[i];
        if (needed) active.push_back(n);
    }
    if (active.empty()) throw_error(DMX_ERR_SHAPE, "no network covers any requested stem");
    std::vector<float> totals(S, 0.0f);
    if (bag) {
        for (int n : active)
            for (int i = 0; i < S; ++i)
                if (bag_weights[n * S + i] != 0.0f && requested[i]) totals[i] += bag_weights[n * S + i];
        for (int i = 0; i < S; ++i)
            if (requested[i] && totals[i] == 0.0f)
                throw_error(DMX_ERR_SHAPE, "no network covers stem index " + std::to_string(i));
    }
    // Per-net masked weights and the totals, on device.
    DBuf d_w = fbuf(s, (int64_t)n_nets * S), d_tot = fbuf(s, S);
    std::vector<float> masked(n_nets * S, 0.0f);
    if (bag)
        for (int n = 0; n < n_nets; ++n)
            for (int i = 0; i < S; ++i) masked[n * S + i] = requested[i] ? bag_weights[n * S + i] : 0.0f;
    DMX_HIP(hipMemcpyAsync(d_w.p, masked.data(), masked.size() * sizeof(float), hipMemcpyHostToDevice, s));
    DMX_HIP(hipMemcpyAsync(d_tot.p, totals.data(), totals.size() * sizeof(float), hipMemcpyHostToDevice, s));
    DBuf d_mask(s, S);
    DMX_HIP(hipMemcpyAsync(d_mask.p, requested.data(), S, hipMemcpyHostToDevice, s));
    // The three copies above read pageable host vectors that end with this
    // call; they are small, and a pageable async copy has read its source
    // when it returns.

    DBuf stats = dbuf(s, 2);
    mix_moments(s, mix, samples, stats.d());
    const float *weight = ola_weight_for(r0, seg, o.transition_power);
    const int64_t max_shift = (int64_t)(0.5 * (double)r0.cfg.samplerate);
    ShiftRng rng(0x5eed1234ULL);
    const int shifts = std::max(0, o.shifts);
    const int passes = std::max(1, shifts);
    // Progress: chunks per pass x passes x active networks.
    auto chunks_in = [&](int64_t view_len) { return (view_len + stride - 1) / stride; };
    total = 0;
    {
        ShiftRng probe(0x5eed1234ULL);
        for (int p = 0; p < passes; ++p) {
            int64_t vl = shifts == 0 ? samples : samples + max_shift - probe.randint(max_shift);
            total += (size_t)chunks_in(vl) * active.size();
        }
    }
    marks.clear();
    size_t done = 0;
    const float scale = shifts > 0 ? 1.0f / (float)shifts : 1.0f;
    if (shifts > 1) {
        // stems accumulates the passes; clear the wanted rows first.
        for (int i = 0; i < S; ++i)
            if (requested[i]) zero_floats(s, stems + (int64_t)i * 2 * samples, 2 * samples);
    }
    const uint8_t *row_mask = static_cast<const uint8_t *>(d_mask.p);
    for (int pass = 0; pass < passes; ++pass) {
        const bool last_pass = pass == passes - 1;
        // mode of ola_finish (pipeline.hip): the only pass, an earlier pass
        // of several, or the last of several.
        const int mode = passes == 1 ? 0 : last_pass ? 2 : 1;
        int64_t offset = 0, view_len = samples, trim = 0, mshift = 0;
        if (shifts > 0) {
            offset = rng.randint(max_shift);
            trim = max_shift - offset;
            view_len = samples + max_shift - offset;
            mshift = max_shift;
        }
        DBuf acc = fbuf(s, (int64_t)rows * view_len), sum_w = fbuf(s, view_len);
        zero_floats(s, acc.f(), (int64_t)rows * view_len);
        zero_floats(s, sum_w.f(), view_len);
        // Chunk groups alternate between two lanes, (stream, side) and
        // (stream_b, side_b), so the forwards of consecutive groups overlap;
        // every overlap-add stays on s in group order. A lane's buffers come
        // from s's pool (taken here, released after the pass) and lane b
        // waits for s before it reuses them.
        const bool two_lanes = r0.stream_b && !single_stream_env() && !r0.trace.record;
        const int lanes = two_lanes ? 2 : 1;
        std::vector<DBuf> chunk, out, one;
        for (int l = 0; l < lanes; ++l) {
            chunk.push_back(fbuf(s, (int64_t)group * 2 * seg));
            out.push_back(fbuf(s, (int64_t)group * rows * seg));
            one.push_back(bag ? fbuf(s, (int64_t)group * rows * seg) : DBuf());
        }
        // ev_lane marks when lane b's buffers are free: first after the
        // pass set-up above, then after each of lane b's overlap-adds.
        if (two_lanes) DMX_HIP(hipEventRecord(r0.ev_lane, s));
        // Lane 1's groups start when the previous lane-0 group reaches a
        // point of its forward (`stagger_default`): 1 = before the
        // transformer, 2 = after it, 10 + i = after encoder level i, 20 + i =
        // after frequency decoder level i, 30 + i = after transformer layer
        // i; 0 = at once. With the stems staying in HBM, starting at once is
        // best (30.7 ms against 31.0 ms when starting at the transformer, on
        // the 60 s separation with the plane linears and attention). When the
        // stems go back to the host, a later start lets the first group end
        // early enough for its readback to overlap the second group's work.
        // DMX_LANE_STAGGER overrides the point, for tuning.
        const char *stag_env = std::getenv("DMX_LANE_STAGGER");
        const int stagger = !two_lanes ? 0 : stag_env ? std::atoi(stag_env) : stagger_default;
        bool mid_marked = false;
        int lane = 0;
        int64_t finished = 0;  // output samples [0, finished) are final (last pass)
        for (int64_t cursor = 0; cursor < view_len;) {
            std::vector<int64_t> starts, lens;
            while ((int)starts.size() < group && cursor < view_len) {
                starts.push_back(cursor);
                lens.push_back(std::min(view_len - cursor, seg));
                cursor += stride;
            }
            const int g = (int)starts.size();
            const hipStream_t ls = lane ? r0.stream_b : s;
            if (lane) DMX_HIP(hipStreamWaitEvent(ls, r0.ev_lane, 0));
            if (lane && mid_marked) DMX_HIP(hipStreamWaitEvent(ls, r0.ev_mid, 0));
            r0.mark_mid = lane == 0 ? stagger : 0;
            mid_marked = lane == 0 && stagger != 0;
            float *chunk_p = chunk[lane].f(), *out_p = out[lane].f(), *one_p = one[lane].f();
            build_chunks(ls, mix, samples, stats.d(), g, starts.data(), lens.data(), seg, view_len, offset, mshift,
                         chunk_p);
            if (!bag) {
                forward_device(r0, ls, chunk_p, g, 2, seg, out_p);
            } else {
                zero_floats(ls, out_p, (int64_t)g * rows * seg);
                for (int n : active) {
                    forward_device(*nets[n], ls, chunk_p, g, 2, seg, one_p);
                    bag_accumulate(ls, one_p, g, S, 2 * seg, d_w.f() + n * S, out_p, 0);
                }
                bag_divide(ls, out_p, g, S, 2 * seg, d_tot.f());
            }
            if (lane) {
                DMX_HIP(hipEventRecord(r0.ev_join, ls));
                DMX_HIP(hipStreamWaitEvent(s, r0.ev_join, 0));
            }
            ola_accumulate(s, out_p, g, starts.data(), lens.data(), seg, rows, view_len, weight, acc.f(), sum_w.f());
            if (lane) DMX_HIP(hipEventRecord(r0.ev_lane, s));
            done += (size_t)g * active.size();
            // No later chunk starts before `cursor`, so view samples below it
            // are final: in the last pass, finish their output samples now,
            // which lets a caller read them back while later groups compute.
            GroupMark m{nullptr, done, finished, finished};
            if (last_pass) {
                const int64_t hi = cursor < view_len ? std::min(samples, std::max<int64_t>(0, cursor - trim)) : samples;
                if (hi > finished) {
                    ola_finish(s, acc.f(), sum_w.f(), rows, view_len, trim, finished, hi, samples, stats.d(), scale,
                               mode, stems, row_mask);
                    if (on_final) on_final(finished, hi);
                    m.hi = finished = hi;
                }
            }
            m.ev = mark_event(r0, marks.size());
            DMX_HIP(hipEventRecord(m.ev, s));
            marks.push_back(m);
            lane = (lane + 1) % lanes;
        }
        r0.mark_mid = 0;
        if (!last_pass)
            ola_finish(s, acc.f(), sum_w.f(), rows, view_len, trim, 0, samples, samples, stats.d(), scale, mode, stems,
                       row_mask);
    }
}

}  // namespace
}  // namespace dmx

namespace dmx {
std::string &last_error_slot() {
    static thread_local std::string slot;
    return slot;
}
}  // namespace dmx

namespace dmx {
namespace {

// dmx_separate and dmx_separate_emit: the mix goes up through the runner's
// pinned staging, the chunk loop runs on the device, and each finished
// region of the stems comes back into pinned memory while later groups
// compute (the OlaRing flush after each segment, streaming.rs:96-261,
// :389-394). Then either a thread of the call copies each region into
// `stems_out` as soon as its readback lands, or the calling thread hands
// each region to `emit` in order.
int host_separation(dmx_runner *const *nets, const float *bag_weights, int32_t n_nets, const uint8_t *stems_wanted,
                    const float *left, const float *right, int64_t samples, int32_t sample_rate,
                    const dmx_separate_options *opts, dmx_progress_fn progress, void *user, float *stems_out,
                    dmx_emit_fn emit, void *emit_user) {
    std::vector<uint64_t> host_jobs;  // pool jobs that touch the caller's memory
    int rc = guarded([&] {
        if (!nets || !nets[0] || !left || !right) throw_error(DMX_ERR_ARGUMENT, "null argument");
        if (samples <= 0) throw_error(DMX_ERR_SHAPE, "empty mix");
        dmx_separate_options o;
        dmx_separate_options_default(&o);
        if (opts) o = *opts;
        dmx_runner &r = *nets[0];
        set_device(&r);
        hipStream_t s = r.stream;
        const int S = r.cfg.sources;
        // Runs of consecutive wanted stems: one 2-D copy each.
        std::vector<std::pair<int, int>> runs;
        for (int i = 0; i < S; ++i) {
            if (stems_wanted && !stems_wanted[i]) continue;
            if (!runs.empty() && runs.back().first + runs.back().second == i)
                ++runs.back().second;
            else
                runs.push_back({i, 1});
        }
        const size_t row_bytes = (size_t)samples * sizeof(float);
        const size_t need = (size_t)(2 + 2 * S) * row_bytes;
        const bool staged = need <= pinned_limit();
        DBuf mix = fbuf(s, 2 * samples), stems = fbuf(s, (int64_t)S * 2 * samples);
        try {
            float *pin_mix = nullptr, *pin_stems = nullptr;
            if (staged) {
                // Everything on the runner's main stream, in order: the mix
                // goes up piece by piece (a piece's host copy overlaps the
                // previous piece's DMA), and each group's finished samples
                // come back into pinned memory as soon as they are final.
                pin_mix = reinterpret_cast<float *>(r.staging.reserve(need));
                pin_stems = pin_mix + 2 * samples;
                const int64_t piece = 1 << 20;
                const float *src[2] = {left, right};
                for (int ch = 0; ch < 2; ++ch)
                    for (int64_t off = 0; off < samples; off += piece) {
                        const int64_t n = std::min(piece, samples - off);
                        float *p = pin_mix + ch * samples + off;
                        host_copy(p, src[ch] + off, (size_t)n * sizeof(float));
                        DMX_HIP(hipMemcpyAsync(mix.f() + ch * samples + off, p, (size_t)n * sizeof(float),
                                               hipMemcpyHostToDevice, s));
                    }
            } else {
                r.ring.upload({{mix.f(), const_cast<float *>(left), row_bytes},
                               {mix.f() + samples, const_cast<float *>(right), row_bytes}},
                              s);
            }
            // Map the caller's output pages on the host threads while the GPU
            // works (queued after the upload's copies; the pool runs jobs in
            // order).
            if (stems_out)
                for (const auto &run : runs)
                    host_jobs.push_back(prefault_async(stems_out + (int64_t)run.first * 2 * samples,
                                                       (size_t)run.second * 2 * row_bytes));
            // Each finished region goes back in up to three blocks (at least
            // 4 MB each): a block's host copy overlaps the next block's DMA,
            // and every block costs one more gap between DMA commands. With
            // `stems_out`, a thread of the call waits for each block and runs
            // its host copies, so they start while this thread is still
            // enqueueing.
            EventCopier copier(r.device, host_jobs);
            struct Block {
                hipEvent_t ev;
                int64_t lo, hi;
            };
            std::vector<Block> blocks;
            const int64_t wanted_rows = [&] {
                int64_t n = 0;
                for (const auto &run : runs) n += 2 * run.second;
                return std::max<int64_t>(n, 1);
            }();
            auto on_final = [&](int64_t lo, int64_t hi) {
                const int64_t min_block = std::max<int64_t>(1 << 14, (int64_t)(4u << 20) / (wanted_rows * 4));
                const int64_t nb = std::max<int64_t>(1, std::min<int64_t>(3, (hi - lo) / min_block));
                for (int64_t i = 0; i < nb; ++i) {
                    const int64_t a = lo + (hi - lo) * i / nb, b = lo + (hi - lo) * (i + 1) / nb;
                    std::vector<Copy> copies;
                    for (const auto &run : runs) {
                        const int64_t at = (int64_t)run.first * 2 * samples + a;
                        DMX_HIP(hipMemcpy2DAsync(pin_stems + at, row_bytes, stems.f() + at, row_bytes,
                                                 (size_t)(b - a) * sizeof(float), (size_t)run.second * 2,
                                                 hipMemcpyDeviceToHost, s));
                        if (stems_out)
                            for (int row = 0; row < 2 * run.second; ++row)
                                copies.push_back({stems_out + at + (int64_t)row * samples,
                                                  pin_stems + at + (int64_t)row * samples,
                                                  (size_t)(b - a) * sizeof(float)});
                    }
                    Block bl{xfer_event(r, blocks.size()), a, b};
                    DMX_HIP(hipEventRecord(bl.ev, s));
                    blocks.push_back(bl);
                    if (stems_out) copier.push(bl.ev, std::move(copies));
                }
            };
            // Rows handed to `emit`: wanted stems' rows, null for the others.
            std::vector<const float *> rows(2 * S, nullptr);
            auto emit_rows = [&](const float *base, int64_t row_stride, int64_t lo, int64_t hi) {
                for (const auto &run : runs)
                    for (int row = 2 * run.first; row < 2 * (run.first + run.second); ++row)
                        rows[row] = base + (int64_t)row * row_stride;
                if (emit(lo, hi - lo, rows.data(), emit_user) != 0)
                    throw_error(DMX_ERR_IO, "the emit callback stopped the separation at sample " + std::to_string(lo));
            };
            std::vector<GroupMark> marks;
            size_t total = 0;
            try {
                // The second lane's group starts after the first group's
                // third transformer layer: the first group then ends early
                // enough for its readback (66 MB of a 60 s mix's 85 MB of
                // stems) to overlap the second group's work (33.6-34.0 ms
                // per 60 s call, against 35.2-35.4 ms with the second lane
                // starting at once, dmx_separate_device's schedule).
                if (staged)
                    separate_device(nets, bag_weights, n_nets, stems_wanted, mix.f(), samples, sample_rate, o,
                                    stems.f(), marks, total, 32, on_final);
                else
                    separate_device(nets, bag_weights, n_nets, stems_wanted, mix.f(), samples, sample_rate, o,
                                    stems.f(), marks, total);
                // Progress after each group, and (emit) each readback block
                // once it has landed, in order, on this thread.
                size_t bi = 0;
                for (const GroupMark &m : marks) {
                    if (emit)
                        for (; bi < blocks.size() && blocks[bi].hi <= m.hi; ++bi) {
                            DMX_HIP(hipEventSynchronize(blocks[bi].ev));
                            emit_rows(pin_stems + blocks[bi].lo, samples, blocks[bi].lo, blocks[bi].hi);
                        }
                    if (progress) {
                        DMX_HIP(hipEventSynchronize(m.ev));
                        progress(m.done, total, user);
                    }
                }
            } catch (...) {
                // No host copy may outlive the call that owns its destination.
                for (hipStream_t st : {r.stream, r.side, r.stream_b, r.side_b}) (void)hipStreamSynchronize(st);
                try {
                    copier.finish();
                } catch (...) {
                }
                throw;
            }
            copier.finish();
            if (!staged) {
                if (stems_out) {
                    std::vector<Span> spans;
                    for (const auto &run : runs) {
                        const int64_t at = (int64_t)run.first * 2 * samples;
                        spans.push_back({stems.f() + at, stems_out + at, (size_t)run.second * 2 * row_bytes});
                    }
                    r.ring.download(spans, s);
                } else {
                    // Too long for the pinned staging: the regions go out
                    // after the chunk loop, a block of rows at a time.
                    DMX_HIP(hipStreamSynchronize(s));
                    const int64_t block = std::max<int64_t>(1 << 14, (int64_t)(8u << 20) / (wanted_rows * 4));
                    std::vector<float> host((size_t)(2 * S) * (size_t)std::min(block, samples));
                    for (int64_t lo = 0; lo < samples; lo += block) {
                        const int64_t n = std::min(block, samples - lo);
                        for (const auto &run : runs)
                            DMX_HIP(hipMemcpy2D(host.data() + (size_t)(2 * run.first) * n, (size_t)n * sizeof(float),
                                                stems.f() + (int64_t)run.first * 2 * samples + lo, row_bytes,
                                                (size_t)n * sizeof(float), (size_t)run.second * 2,
                                                hipMemcpyDeviceToHost));
                        emit_rows(host.data(), n, lo, lo + n);
                    }
                }
            }
            DMX_HIP(hipStreamSynchronize(s));
        } catch (...) {
            // The device buffers go back to the pool: let nothing use them.
            for (hipStream_t st : {r.stream, r.side, r.stream_b, r.side_b}) (void)hipStreamSynchronize(st);
            throw;
        }
    });
    for (uint64_t t : host_jobs) HostPool::instance().wait(t);
    return rc;
}

}  // namespace
}  // namespace dmx

using namespace dmx;

extern "C" {

void dmx_config_default(dmx_config *c) {
    if (!c) return;
    c->sources = 4;
    c->audio_channels = 2;
    c->samplerate = 44100;
    c->segment = 39.0 / 5.0;
    c->channels = 48;
    c->growth = 2;
    c->nfft = 4096;
    c->depth = 4;
    c->stride = 4;
    c->kernel_size = 8;
    c->context = 1;
    c->freq_emb = 0.2;
    c->emb_scale = 10.0;
    c->cac = 1;
    c->bottom_channels = 512;
    c->t_layers = 5;
    c->t_heads = 8;
    c->t_hidden_scale = 4.0;
    c->t_max_period = 10000.0;
    c->t_weight_pos_embed = 1.0;
}

int64_t dmx_config_training_length(const dmx_config *c) {
    return c ? (int64_t)(c->segment * (double)c->samplerate) : 0;
}

const char *dmx_last_error(void) { return last_error_slot().c_str(); }

int dmx_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

int dmx_runner_create(const dmx_tensor *weights, size_t n_weights, const dmx_config *cfg, int device_ordinal,
                      int precision, dmx_runner **out) {
    if (!out) {
        last_error_slot() = "null output pointer";
        return DMX_ERR_ARGUMENT;
    }
    *out = nullptr;
    std::unique_ptr<dmx_runner> r(new dmx_runner());
    int rc = guarded([&] {
        if (!weights || !cfg) throw_error(DMX_ERR_ARGUMENT, "null weights or config");
        if (precision != DMX_PRECISION_FP32 && precision != DMX_PRECISION_BF16 &&
            precision != DMX_PRECISION_FP32_MFMA)
            throw_error(DMX_ERR_ARGUMENT, "unknown precision");
        validate(*cfg);
        int count = 0;
        if (hipGetDeviceCount(&count) != hipSuccess || count == 0) throw_error(DMX_ERR_GPU, "no HIP device is visible");
        if (device_ordinal < 0 || device_ordinal >= count)
            throw_error(DMX_ERR_GPU, "device ordinal " + std::to_string(device_ordinal) + " out of range");
        r->cfg = *cfg;
        r->device = device_ordinal;
        r->precision = precision;
        {
            MfmaPrecisionScope prec(mfma_of_precision(precision));
            r->planes = linear_planes();
        }
        r->training_length = dmx_config_training_length(cfg);
        r->hop = cfg->nfft / 4;
        DMX_HIP(hipSetDevice(device_ordinal));
        hipDeviceProp_t prop;
        DMX_HIP(hipGetDeviceProperties(&prop, device_ordinal));
        r->tag = std::string("hip:") + prop.name + ":" + prop.gcnArchName;
        DMX_HIP(hipStreamCreateWithFlags(&r->stream, hipStreamNonBlocking));
        DMX_HIP(hipStreamCreateWithFlags(&r->side, hipStreamNonBlocking));
        DMX_HIP(hipStreamCreateWithFlags(&r->stream_b, hipStreamNonBlocking));
        DMX_HIP(hipStreamCreateWithFlags(&r->side_b, hipStreamNonBlocking));
        DMX_HIP(hipEventCreateWithFlags(&r->ev_fork, hipEventDisableTiming));
        DMX_HIP(hipEventCreateWithFlags(&r->ev_join, hipEventDisableTiming));
        DMX_HIP(hipEventCreateWithFlags(&r->ev_lane, hipEventDisableTiming));
        DMX_HIP(hipEventCreateWithFlags(&r->ev_mid, hipEventDisableTiming));
        load_weights(*r, weights, n_weights);
        // Tables made by kernels at load time are ready before any stream uses them.
        DMX_HIP(hipStreamSynchronize(r->stream));
    });
    if (rc != DMX_OK) {
        for (hipEvent_t e : {r->ev_fork, r->ev_join, r->ev_lane, r->ev_mid})
            if (e) (void)hipEventDestroy(e);
        for (hipStream_t st : {r->side, r->stream_b, r->side_b, r->stream})
            if (st) (void)hipStreamDestroy(st);
        if (r->weight_mem) (void)hipFree(r->weight_mem);
        for (void *p : r->owned) (void)hipFree(p);
        return rc;
    }
    *out = r.release();
    return DMX_OK;
}

void dmx_runner_destroy(dmx_runner *r) {
    if (!r) return;
    (void)hipSetDevice(r->device);
    for (hipStream_t st : {r->stream, r->side, r->stream_b, r->side_b})
        if (st) {
            (void)hipStreamSynchronize(st);
            StreamPool::instance().trim(st);
        }
    if (r->weight_mem) (void)hipFree(r->weight_mem);
    for (void *p : r->owned) (void)hipFree(p);
    for (hipEvent_t e : {r->ev_fork, r->ev_join, r->ev_lane, r->ev_mid})
        if (e) (void)hipEventDestroy(e);
    for (hipEvent_t e : r->marks) (void)hipEventDestroy(e);
    for (hipEvent_t e : r->xfer) (void)hipEventDestroy(e);
    for (PendingSlot &sl : r->pending) {
        if (sl.done) (void)hipEventDestroy(sl.done);
        if (sl.in) (void)hipHostFree(sl.in);
        if (sl.out) (void)hipHostFree(sl.out);
    }
    for (hipStream_t st : {r->side, r->stream_b, r->side_b, r->stream})
        if (st) (void)hipStreamDestroy(st);
    delete r;
}

const char *dmx_runner_backend_tag(const dmx_runner *r) { return r ? r->tag.c_str() : ""; }
void *dmx_runner_stream(dmx_runner *r) { return r ? (void *)r->stream : nullptr; }

int dmx_synchronize(dmx_runner *r) {
    return guarded([&] {
        if (!r) throw_error(DMX_ERR_ARGUMENT, "null runner");
        set_device(r);
        // dmx_forward_start may have queued a group on the second lane.
        for (hipStream_t st : {r->stream, r->side, r->stream_b, r->side_b})
            if (st) DMX_HIP(hipStreamSynchronize(st));
    });
}

int dmx_set_trace(dmx_runner *r, dmx_trace_wants_fn wants, dmx_trace_record_fn record, void *user) {
    return guarded([&] {
        if (!r) throw_error(DMX_ERR_ARGUMENT, "null runner");
        r->trace = Trace{wants, record, user};
    });
}

int dmx_forward_device(dmx_runner *r, const float *d_mix, int64_t batch, int64_t channels, int64_t length,
                       float *d_stems) {
    return guarded([&] {
        if (!r || !d_mix || !d_stems) throw_error(DMX_ERR_ARGUMENT, "null argument");
        set_device(r);
        forward_device(*r, r->stream, d_mix, batch, channels, length, d_stems);
    });
}

int dmx_forward_start(dmx_runner *r, const float *mix, int64_t batch, int64_t channels, int64_t length,
                      dmx_pending **out) {
    if (out) *out = nullptr;
    return guarded([&] {
        if (!r || !mix || !out) throw_error(DMX_ERR_ARGUMENT, "null argument");
        set_device(r);
        if (channels != r->cfg.audio_channels) throw_error(DMX_ERR_SHAPE, "wrong audio channel count");
        if (batch <= 0 || length <= 0 || length > r->training_length)
            throw_error(DMX_ERR_SHAPE, "input must hold 1..training_length samples per channel");
        const size_t in_n = (size_t)(batch * channels * length);
        const size_t out_n = (size_t)(batch * r->cfg.sources * channels * length);
        // A free staging slot: one that is large enough, else any free one
        // (grown), else a new one. Two groups in flight use two slots.
        int k = -1;
        for (int i = 0; i < (int)r->pending.size() && k < 0; ++i)
            if (!r->pending[i].busy && r->pending[i].in_cap >= in_n && r->pending[i].out_cap >= out_n) k = i;
        for (int i = 0; i < (int)r->pending.size() && k < 0; ++i)
            if (!r->pending[i].busy) k = i;
        if (k < 0) {
            r->pending.emplace_back();
            k = (int)r->pending.size() - 1;
            DMX_HIP(hipEventCreateWithFlags(&r->pending[k].done, hipEventDisableTiming));
        }
        PendingSlot &sl = r->pending[k];
        if (sl.in_cap < in_n) {
            if (sl.in) DMX_HIP(hipHostFree(sl.in));
            sl.in = nullptr;
            sl.in_cap = 0;
            DMX_HIP(hipHostMalloc((void **)&sl.in, in_n * sizeof(float), hipHostMallocDefault));
            sl.in_cap = in_n;
        }
        if (sl.out_cap < out_n) {
            if (sl.out) DMX_HIP(hipHostFree(sl.out));
            sl.out = nullptr;
            sl.out_cap = 0;
            DMX_HIP(hipHostMalloc((void **)&sl.out, out_n * sizeof(float), hipHostMallocDefault));
            sl.out_cap = out_n;
        }
        // Consecutive groups alternate between the two stream pairs, so the
        // group queued ahead runs beside the one being collected.
        const bool two_lanes = r->stream_b && !r->trace.record && !single_stream_env();
        hipStream_t ls = two_lanes && (r->next_lane++ & 1) ? r->stream_b : r->stream;
        host_copy(sl.in, mix, in_n * sizeof(float));
        try {
            DBuf d_in(ls, in_n * sizeof(float)), d_out(ls, out_n * sizeof(float));
            DMX_HIP(hipMemcpyAsync(d_in.p, sl.in, in_n * sizeof(float), hipMemcpyHostToDevice, ls));
            forward_device(*r, ls, d_in.f(), batch, channels, length, d_out.f());
            DMX_HIP(hipMemcpyAsync(sl.out, d_out.p, out_n * sizeof(float), hipMemcpyDeviceToHost, ls));
            DMX_HIP(hipEventRecord(sl.done, ls));
        } catch (...) {
            // Nothing queued may still read or write the slot once it is free.
            (void)hipStreamSynchronize(ls);
            throw;
        }
        sl.busy = true;
        *out = new dmx_pending{r, k, out_n};
    });
}

int dmx_forward_collect(dmx_runner *r, dmx_pending *p, float *stems) {
    // An argument error leaves the group pending; any other outcome ends it.
    if (!r || !p || !stems) {
        last_error_slot() = "null argument";
        return DMX_ERR_ARGUMENT;
    }
    if (p->runner != r) {
        last_error_slot() = "the pending group belongs to another runner";
        return DMX_ERR_ARGUMENT;
    }
    PendingSlot &sl = r->pending[p->slot];
    int rc = guarded([&] {
        set_device(r);
        DMX_HIP(hipEventSynchronize(sl.done));
        advise_huge_pages(stems, p->count * sizeof(float));
        host_copy(stems, sl.out, p->count * sizeof(float));
    });
    (void)hipEventSynchronize(sl.done);
    sl.busy = false;
    delete p;
    return rc;
}

int dmx_forward(dmx_runner *r, const float *mix, int64_t batch, int64_t channels, int64_t length, float *stems) {
    dmx_pending *p = nullptr;
    int rc = dmx_forward_start(r, mix, batch, channels, length, &p);
    if (rc != DMX_OK) return rc;
    return dmx_forward_collect(r, p, stems);
}

int dmx_crosstransformer_device(dmx_runner *r, const float *d_spec, const float *d_time, int64_t batch, int64_t freqs,
                                int64_t frames, int64_t time_len, float *d_spec_out, float *d_time_out) {
    return guarded([&] {
        if (!r || !d_spec || !d_time || !d_spec_out || !d_time_out) throw_error(DMX_ERR_ARGUMENT, "null argument");
        if (batch <= 0 || freqs <= 0 || frames <= 0 || time_len <= 0) throw_error(DMX_ERR_SHAPE, "empty input");
        set_device(r);
        transformer_only(*r, r->stream, d_spec, d_time, (int)batch, (int)freqs, (int)frames, (int)time_len,
                         d_spec_out, d_time_out);
    });
}

void dmx_separate_options_default(dmx_separate_options *o) {
    if (!o) return;
    o->shifts = 1;
    o->overlap = 0.25;
    o->transition_power = 1.0;
    o->segment = 0.0;
    o->batch_chunks = 1;
}

int dmx_separate_device(dmx_runner *const *nets, const float *bag_weights, int32_t n_nets, const uint8_t *stems_wanted,
                        const float *d_mix, int64_t samples, int32_t sample_rate, const dmx_separate_options *opts,
                        dmx_progress_fn progress, void *user, float *d_stems) {
    return guarded([&] {
        if (!nets || !nets[0] || !d_mix || !d_stems) throw_error(DMX_ERR_ARGUMENT, "null argument");
        dmx_separate_options o;
        dmx_separate_options_default(&o);
        if (opts) o = *opts;
        set_device(nets[0]);
        std::vector<GroupMark> marks;
        size_t total = 0;
        separate_device(nets, bag_weights, n_nets, stems_wanted, d_mix, samples, sample_rate, o, d_stems, marks,
                        total);
        // Progress comes from the host waiting on each group's mark, so a
        // callback does not change the schedule on the GPU.
        if (progress)
            for (const GroupMark &m : marks) {
                DMX_HIP(hipEventSynchronize(m.ev));
                progress(m.done, total, user);
            }
    });
}

int dmx_separate(dmx_runner *const *nets, const float *bag_weights, int32_t n_nets, const uint8_t *stems_wanted,
                 const float *left, const float *right, int64_t samples, int32_t sample_rate,
                 const dmx_separate_options *opts, dmx_progress_fn progress, void *user, float *stems_out) {
    if (!stems_out) return guarded([] { throw_error(DMX_ERR_ARGUMENT, "null argument"); });
    return host_separation(nets, bag_weights, n_nets, stems_wanted, left, right, samples, sample_rate, opts, progress,
                           user, stems_out, nullptr, nullptr);
}

int dmx_separate_emit(dmx_runner *const *nets, const float *bag_weights, int32_t n_nets, const uint8_t *stems_wanted,
                      const float *left, const float *right, int64_t samples, int32_t sample_rate,
                      const dmx_separate_options *opts, dmx_progress_fn progress, void *user, dmx_emit_fn emit,
                      void *emit_user) {
    if (!emit) return guarded([] { throw_error(DMX_ERR_ARGUMENT, "null emit callback"); });
    return host_separation(nets, bag_weights, n_nets, stems_wanted, left, right, samples, sample_rate, opts, progress,
                           user, nullptr, emit, emit_user);
}

}  // extern "C"
