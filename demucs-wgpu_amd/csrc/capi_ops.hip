// capi_ops.hip — include/dmx_ops.h: one kernel (group) per call, on the
// caller's stream, for the parity tests.
#include <hip/hip_runtime.h>

#include <map>
#include <memory>
#include <mutex>
#include <vector>

#include "../../include/dmx_ops.h"
#include "common.h"
#include "ops.h"

using namespace dmx;

namespace {

hipStream_t as_stream(void *s) { return static_cast<hipStream_t>(s); }

// Twiddles + window for nfft 4096, uploaded once per process (per device 0 context).
const float *twiddles_4096() {
    static float *d = nullptr;
    if (!d) {
        std::vector<float> h(4096 / 2 * 2 + 4096);
        make_twiddles(4096, h.data());
        DMX_HIP(hipMalloc(&d, h.size() * sizeof(float)));
        DMX_HIP(hipMemcpy(d, h.data(), h.size() * sizeof(float), hipMemcpyHostToDevice));
    }
    return d;
}

struct Scratch {
    void *p = nullptr;
    explicit Scratch(size_t bytes) { DMX_HIP(hipMalloc(&p, std::max<size_t>(bytes, 16))); }
    ~Scratch() { (void)hipFree(p); }
};

// A device conv weight (oc, ic, kh, kw) in GEMM order (conv_gemm_weights):
// the weight itself when that is its PyTorch layout, else a repacked copy
// held by `keep` (the caller synchronises before `keep` goes).
const float *gemm_weights(hipStream_t s, const float *w, int oc, int ic, int kh, int kw,
                          std::unique_ptr<Scratch> &keep) {
    if (!conv_tap_major(ic, kh, kw)) return w;
    require_ptrs({w}, "conv weight");
    const size_t n = (size_t)oc * ic * kh * kw;
    std::vector<float> h(n), g(n);
    DMX_HIP(hipStreamSynchronize(s));
    DMX_HIP(hipMemcpy(h.data(), w, n * sizeof(float), hipMemcpyDeviceToHost));
    conv_gemm_weights(h.data(), oc, ic, kh, kw, g.data());
    keep = std::make_unique<Scratch>(n * sizeof(float));
    DMX_HIP(hipMemcpy(keep->p, g.data(), n * sizeof(float), hipMemcpyHostToDevice));
    return static_cast<const float *>(keep->p);
}

// ---- fixed scratch of dmx_op_spec_normalise_noalloc ----
// Layout: the 4096-point twiddles and periodic Hann window (8192 floats),
// then the f64 moments (4 per batch row), then the STFT frames
// (batch x frames x 2 channels x 2048 bins x complex).
constexpr int NOALLOC_MAX_BATCH = 64;
constexpr int64_t NOALLOC_MAX_FRAMES = 672;  // batch x ceil(L / 1024): two 7.8 s segments
constexpr size_t NOALLOC_TW_BYTES = (size_t)(4096 + 4096) * sizeof(float);
constexpr size_t NOALLOC_STATS_BYTES = (size_t)4 * NOALLOC_MAX_BATCH * sizeof(double);
constexpr size_t NOALLOC_FRAME_FLOATS = (size_t)2 * 2048 * 2;
constexpr size_t NOALLOC_BYTES =
    NOALLOC_TW_BYTES + NOALLOC_STATS_BYTES + (size_t)NOALLOC_MAX_FRAMES * NOALLOC_FRAME_FLOATS * sizeof(float);
static_assert(NOALLOC_TW_BYTES % 256 == 0 && NOALLOC_STATS_BYTES % 256 == 0, "scratch sections stay 256-B aligned");

}  // namespace

// Each GPU holds its own copy (about 22 MB) from the library's load until the
// process ends. Host code never uses this name as an address: the per-device
// address comes from hipGetSymbolAddress (scratch_on_current_device).
static __device__ __align__(256) unsigned char scratch[NOALLOC_BYTES];

namespace {

// The current device's address of `scratch`; the first call on a device also
// writes the twiddle table into it (a synchronous copy, no allocation).
unsigned char *scratch_on_current_device() {
    static std::mutex mu;
    static std::map<int, unsigned char *> ptrs;
    int dev = -1;
    DMX_HIP(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(mu);
    auto it = ptrs.find(dev);
    if (it != ptrs.end()) return it->second;
    void *p = nullptr;
    DMX_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) throw Error(6, "hipGetSymbolAddress returned no address for the fixed scratch");
    std::vector<float> tw(NOALLOC_TW_BYTES / sizeof(float));
    make_twiddles(4096, tw.data());
    DMX_HIP(hipMemcpy(p, tw.data(), NOALLOC_TW_BYTES, hipMemcpyHostToDevice));
    ptrs[dev] = static_cast<unsigned char *>(p);
    return ptrs[dev];
}

}  // namespace

namespace {

// The K/V planes layout of dmx_op_kv_planes for (batch, heads, n_k):
// K planes [3][batch][n_k][D], V^T planes [3][batch * D][ldvt].
KVPlanes op_kv_layout(unsigned short *kp, unsigned short *vtp, int batch, int heads, int n_k) {
    const int64_t D = (int64_t)heads * 64, ldvt = kv_ldvt(n_k);
    KVPlanes kv;
    kv.k = kp;
    kv.vt = vtp;
    kv.ldk = D;
    kv.k_bs = (int64_t)n_k * D;
    kv.k_stride = (int64_t)batch * n_k * D;
    kv.ldvt = ldvt;
    kv.vt_stride = (int64_t)batch * D * ldvt;
    return kv;
}

// Scratch planes of one problem's K and V, filled from fp32 K and V.
struct OpKV {
    std::unique_ptr<Scratch> k, vt;
    KVPlanes kv;
    OpKV(hipStream_t s, const float *kf, const float *vf, int batch, int heads, int n_k) {
        require_ptrs({kf, vf}, "attention");
        const int64_t D = (int64_t)heads * 64;
        DMX_REQUIRE(batch > 0 && heads > 0 && n_k > 0, "attention: empty problem");
        k.reset(new Scratch((size_t)3 * batch * n_k * D * 2));
        vt.reset(new Scratch((size_t)3 * batch * D * kv_ldvt(n_k) * 2));
        kv = op_kv_layout(static_cast<unsigned short *>(k->p), static_cast<unsigned short *>(vt->p), batch, heads, n_k);
        kv_to_planes(s, kf, D, vf, D, (int64_t)n_k * D, batch, heads, n_k, kv);
    }
};

bool op_attention_planes() { return mfma_precision() == MfmaPrecision::FP32X3 && attention_planes_enabled(); }

}  // namespace

extern "C" {

int dmx_op_conv2d(void *stream, const float *x, const float *skip, int b, int ic, int h, int w, const float *weight,
                  const float *bias, int oc, int kh, int kw, int sh, int sw, int ph, int pw, int dh, int dw, int act,
                  float *out) {
    return guarded([&] {
        hipStream_t s = as_stream(stream);
        std::unique_ptr<Scratch> keep;
        const float *wg = gemm_weights(s, weight, oc, ic, kh, kw, keep);
        conv2d(s, x, skip, b, ic, h, w, wg, bias, oc, kh, kw, sh, sw, ph, pw, dh, dw, out, (Act)act);
        if (keep) DMX_HIP(hipStreamSynchronize(s));
    });
}

int dmx_op_conv2d_glu(void *stream, const float *x, const float *skip, int b, int ic, int h, int w,
                      const float *weight, const float *bias, int C, int kh, int kw, int ph, int pw, const float *emb,
                      float emb_scale, float *out) {
    return guarded([&] {
        hipStream_t s = as_stream(stream);
        if (kh == 3 && kw == 3 && ph == 1 && pw == 1 && !emb && winograd_applies(ic, C, h, w)) {
            // The decoder rewrite's shape: the Winograd path the runner takes for it.
            require_ptrs({x, weight, bias, out}, "conv2d_glu");
            std::vector<float> hw((size_t)2 * C * ic * 9), u((size_t)winograd_weight_floats(ic, C));
            DMX_HIP(hipStreamSynchronize(s));
            DMX_HIP(hipMemcpy(hw.data(), weight, hw.size() * sizeof(float), hipMemcpyDeviceToHost));
            winograd_weights(hw.data(), 2 * C, ic, u.data());
            Scratch du(u.size() * sizeof(float)), ws((size_t)winograd_scratch_floats(b, ic, C, h, w) * sizeof(float));
            DMX_HIP(hipMemcpy(du.p, u.data(), u.size() * sizeof(float), hipMemcpyHostToDevice));
            conv3x3_glu_winograd(s, x, skip, b, ic, C, h, w, static_cast<const float *>(du.p), bias, out,
                                 static_cast<float *>(ws.p));
            DMX_HIP(hipStreamSynchronize(s));
            return;
        }
        std::unique_ptr<Scratch> keep;
        const float *wg = gemm_weights(s, weight, 2 * C, ic, kh, kw, keep);
        conv2d_glu(s, x, skip, b, ic, h, w, wg, bias, C, kh, kw, ph, pw, out, emb, emb_scale);
        if (keep) DMX_HIP(hipStreamSynchronize(s));
    });
}

int dmx_op_conv_transpose(void *stream, const float *x, int b, int ic, int A, int P, const float *weight,
                          const float *bias, int oc, int k, int st, int crop, int a_out, int act, float *out) {
    return guarded([&] {
        hipStream_t s = as_stream(stream);
        std::vector<float> hw((size_t)ic * oc * k);
        DMX_HIP(hipStreamSynchronize(s));
        DMX_HIP(hipMemcpy(hw.data(), weight, hw.size() * sizeof(float), hipMemcpyDeviceToHost));
        int taps = conv_transpose_taps(k, st);
        std::vector<float> packed((size_t)st * oc * ic * taps);
        pack_conv_transpose(hw.data(), ic, oc, k, st, packed.data());
        Scratch d(packed.size() * sizeof(float));
        DMX_HIP(hipMemcpy(d.p, packed.data(), packed.size() * sizeof(float), hipMemcpyHostToDevice));
        conv_transpose_axis(s, x, b, ic, A, P, static_cast<float *>(d.p), bias, oc, k, st, crop, a_out, out,
                            (Act)act);
        DMX_HIP(hipStreamSynchronize(s));
    });
}

int dmx_op_dconv_layer(void *stream, float *x, int B, int C, int F, int T, int dilation, const float *w1,
                       const float *b1, int hidden, const float *n1w, const float *n1b, const float *w2,
                       const float *b2, const float *n2w, const float *n2b, const float *gamma) {
    return guarded([&] {
        hipStream_t s = as_stream(stream);
        Scratch h((size_t)dconv_hidden_floats(B * F, hidden, T) * sizeof(float)),
            st((size_t)4 * B * F * sizeof(double));
        std::unique_ptr<Scratch> keep;
        const float *w1g = gemm_weights(s, w1, hidden, C, 1, 3, keep);
        Scratch gram((size_t)dconv_gram_doubles(hidden) * sizeof(double));
        dconv_gram_weights(s, w2, b2, C, hidden, static_cast<double *>(gram.p));
        dconv_layer(s, x, B, C, F, T, dilation, w1, w1g, nullptr, b1, hidden, n1w, n1b, w2, b2, n2w, n2b, gamma,
                    static_cast<const double *>(gram.p), static_cast<float *>(h.p), static_cast<double *>(st.p));
        DMX_HIP(hipStreamSynchronize(s));
    });
}

int dmx_op_dconv(void *stream, float *x, int B, int C, int F, int T, int hidden, const float *const *params) {
    return guarded([&] {
        hipStream_t s = as_stream(stream);
        if (!params) throw std::invalid_argument("dmx_op_dconv: params is null");
        // w1 of each layer as (C*3, H), through the host.
        std::vector<float> hw((size_t)hidden * C * 3), ht(hw.size());
        std::unique_ptr<Scratch> w1t[2];
        DConvRowLayer L[2];
        DMX_HIP(hipStreamSynchronize(s));
        for (int d = 0; d < 2; ++d) {
            const float *const *p = params + 9 * d;
            require_ptrs({p[0], p[1], p[2], p[3], p[4], p[5], p[6], p[7], p[8]}, "dconv weight");
            DMX_HIP(hipMemcpy(hw.data(), p[0], hw.size() * sizeof(float), hipMemcpyDeviceToHost));
            dconv_w1_transposed(hw.data(), C, hidden, ht.data());
            w1t[d] = std::make_unique<Scratch>(ht.size() * sizeof(float));
            DMX_HIP(hipMemcpy(w1t[d]->p, ht.data(), ht.size() * sizeof(float), hipMemcpyHostToDevice));
            L[d] = {static_cast<const float *>(w1t[d]->p), p[1], p[2], p[3], p[4], p[5], p[6], p[7], p[8]};
        }
        if (!dconv_rows(s, x, B, C, F, T, hidden, L)) {
            // Rows too long (or widths the row kernel does not cover): the layers one at a time.
            Scratch h((size_t)dconv_hidden_floats(B * F, hidden, T) * sizeof(float)),
                st((size_t)4 * B * F * sizeof(double));
            for (int d = 0; d < 2; ++d) {
                const float *const *p = params + 9 * d;
                std::unique_ptr<Scratch> keep;
                const float *w1g = gemm_weights(s, p[0], hidden, C, 1, 3, keep);
                Scratch gram((size_t)dconv_gram_doubles(hidden) * sizeof(double));
                dconv_gram_weights(s, p[4], p[5], C, hidden, static_cast<double *>(gram.p));
                dconv_layer(s, x, B, C, F, T, 1 << d, p[0], w1g, L[d].w1_t, p[1], hidden, p[2], p[3], p[4], p[5],
                            p[6], p[7], p[8], static_cast<const double *>(gram.p), static_cast<float *>(h.p),
                            static_cast<double *>(st.p));
                DMX_HIP(hipStreamSynchronize(s));
            }
        }
        DMX_HIP(hipStreamSynchronize(s));
    });
}

int dmx_op_linear(void *stream, const float *x, int rows, int K, const float *w, const float *bias, int N, int tail,
                  const float *residual, const float *gamma, float *out) {
    return guarded([&] {
        hipStream_t s = as_stream(stream);
        const int P = linear_planes();
        if (P > 0 && rows > 0 && N > 0 && K > 0 && K % 64 == 0) {
            // The transformer's plane path: x and W split into P bf16 planes
            // (the runner splits W once at load and has x's producers write
            // planes), then the plane GEMM.
            require_ptrs({x, w}, "linear");
            const int64_t nx = (int64_t)rows * K, nw = (int64_t)N * K;
            const int64_t sx = (nx + 7) / 8 * 8, sw = (nw + 7) / 8 * 8;
            Scratch xp((size_t)sx * P * 2), wp((size_t)sw * P * 2);
            const Planes xpl{static_cast<unsigned short *>(xp.p), sx, P}, wpl{static_cast<unsigned short *>(wp.p), sw, P};
            split_to_planes(s, x, nx, xpl);
            split_to_planes(s, w, nw, wpl);
            linear_planes(s, xpl, K, nx, wpl, bias, 1, rows, K, N, out, Planes{}, N, (int64_t)rows * N,
                          (LinearTail)tail, residual, gamma, nullptr);
            DMX_HIP(hipStreamSynchronize(s));
            return;
        }
        linear(s, x, K, (int64_t)rows * K, w, bias, 1, rows, K, N, out, N, (int64_t)rows * N, (LinearTail)tail,
               residual, gamma, nullptr);
    });
}

int dmx_op_pointwise(void *stream, const float *w, const float *bias, const float *x, int batches, int M, int K,
                     int N, float *out) {
    return guarded([&] { pointwise(as_stream(stream), w, bias, x, batches, M, K, N, out, ACT_NONE); });
}

int dmx_op_attention(void *stream, const float *q, const float *k, const float *v, float *out, int batch, int heads,
                     int n_q, int n_k, float scale) {
    return guarded([&] {
        hipStream_t s = as_stream(stream);
        int64_t D = (int64_t)heads * 64;
        AttentionArgs a{q, D, k, D, v, D, out, D, batch, heads, n_q, n_k, 64, n_q * D, n_k * D, n_q * D};
        if (op_attention_planes()) {
            OpKV kv(s, k, v, batch, heads, n_k);
            a.kv = kv.kv;
            attention_grouped(s, &a, 1, scale);
            DMX_HIP(hipStreamSynchronize(s));
            return;
        }
        attention_grouped(s, &a, 1, scale);
    });
}

int dmx_op_attention_pair(void *stream, const float *q0, const float *k0, const float *v0, float *out0, int n_q0,
                          int n_k0, const float *q1, const float *k1, const float *v1, float *out1, int n_q1,
                          int n_k1, int batch, int heads, float scale) {
    return guarded([&] {
        hipStream_t s = as_stream(stream);
        const int64_t D = (int64_t)heads * 64;
        AttentionArgs p[2] = {
            {q0, D, k0, D, v0, D, out0, D, batch, heads, n_q0, n_k0, 64, n_q0 * D, n_k0 * D, n_q0 * D},
            {q1, D, k1, D, v1, D, out1, D, batch, heads, n_q1, n_k1, 64, n_q1 * D, n_k1 * D, n_q1 * D}};
        if (op_attention_planes()) {
            OpKV kv0(s, k0, v0, batch, heads, n_k0), kv1(s, k1, v1, batch, heads, n_k1);
            p[0].kv = kv0.kv;
            p[1].kv = kv1.kv;
            attention_grouped(s, p, 2, scale);
            DMX_HIP(hipStreamSynchronize(s));
            return;
        }
        attention_grouped(s, p, 2, scale);
    });
}

int dmx_op_kv_planes(void *stream, const float *k, const float *v, int batch, int heads, int n_k,
                     unsigned short *k_planes, unsigned short *vt_planes) {
    return guarded([&] {
        require_ptrs({k, v, k_planes, vt_planes}, "kv_planes");
        DMX_REQUIRE(batch > 0 && heads > 0 && n_k > 0, "kv_planes: empty problem");
        const int64_t D = (int64_t)heads * 64;
        kv_to_planes(as_stream(stream), k, D, v, D, (int64_t)n_k * D, batch, heads, n_k,
                     op_kv_layout(k_planes, vt_planes, batch, heads, n_k));
    });
}

int dmx_op_attention_pair_planes(void *stream, const float *q0, unsigned short *kp0, unsigned short *vtp0,
                                 float *out0, int n_q0, int n_k0, const float *q1, unsigned short *kp1,
                                 unsigned short *vtp1, float *out1, int n_q1, int n_k1, int batch, int heads,
                                 float scale) {
    return guarded([&] {
        const int64_t D = (int64_t)heads * 64;
        AttentionArgs p[2] = {
            {q0, D, nullptr, D, nullptr, D, out0, D, batch, heads, n_q0, n_k0, 64, n_q0 * D, n_k0 * D, n_q0 * D},
            {q1, D, nullptr, D, nullptr, D, out1, D, batch, heads, n_q1, n_k1, 64, n_q1 * D, n_k1 * D, n_q1 * D}};
        p[0].kv = op_kv_layout(kp0, vtp0, batch, heads, n_k0);
        p[1].kv = op_kv_layout(kp1, vtp1, batch, heads, n_k1);
        attention_grouped(as_stream(stream), p, 2, scale);
    });
}

int dmx_op_layer_norm(void *stream, const float *x, int rows, int dim, const float *w, const float *b, float *out) {
    return guarded([&] { layer_norm_rows(as_stream(stream), x, rows, dim, w, b, out, nullptr, 0); });
}

int dmx_op_group_norm(void *stream, const float *x, int b, int c, int inner, int groups, const float *w,
                      const float *bias, float *out) {
    return guarded([&] {
        hipStream_t s = as_stream(stream);
        Scratch st((size_t)2 * b * groups * sizeof(double));
        group_norm(s, x, b, c, inner, groups, w, bias, out, static_cast<double *>(st.p));
        DMX_HIP(hipStreamSynchronize(s));
    });
}

int dmx_op_glu(void *stream, const float *x, int b, int c2, int inner, float *out) {
    return guarded([&] { glu(as_stream(stream), x, b, c2, inner, out); });
}

int dmx_op_set_precision(int precision) {
    return guarded([&] {
        mfma_precision() = mfma_of_precision(precision);
    });
}

int dmx_op_gelu(void *stream, const float *x, int64_t n, float *out) {
    return guarded([&] { gelu(as_stream(stream), x, n, out); });
}

int dmx_op_spec_normalise(void *stream, const float *mix, int b, int L, float *xspec, float *xwave, float *norms) {
    return guarded([&] {
        hipStream_t s = as_stream(stream);
        int le = (L + 1023) / 1024;
        Scratch frames((size_t)b * 2 * le * 2048 * 2 * sizeof(float)), st((size_t)4 * b * sizeof(double));
        spec_and_normalise(s, mix, b, L, 4096, static_cast<float *>(frames.p), xspec, xwave, norms,
                           static_cast<double *>(st.p), twiddles_4096());
        DMX_HIP(hipStreamSynchronize(s));
    });
}

int dmx_op_spec_normalise_noalloc(void *stream, const float *mix, int b, int L, float *xspec, float *xwave,
                                  float *norms) {
    return guarded([&] {
        hipStream_t s = as_stream(stream);
        if (b <= 0 || L <= 0) throw Error(1, "dmx_op_spec_normalise_noalloc: empty input");
        const int64_t frames = (int64_t)b * ceil_div(L, 1024);
        if (b > NOALLOC_MAX_BATCH || frames > NOALLOC_MAX_FRAMES)
            throw Error(1, "dmx_op_spec_normalise_noalloc: batch " + std::to_string(b) + " x " +
                               std::to_string(ceil_div(L, 1024)) + " frames exceeds the fixed scratch (at most " +
                               std::to_string(NOALLOC_MAX_BATCH) + " rows and " + std::to_string(NOALLOC_MAX_FRAMES) +
                               " batch frames, two 7.8 s segments); use dmx_op_spec_normalise");
        unsigned char *base = scratch_on_current_device();
        const float *twiddles = reinterpret_cast<const float *>(base);
        double *stats = reinterpret_cast<double *>(base + NOALLOC_TW_BYTES);
        float *frame_buf = reinterpret_cast<float *>(base + NOALLOC_TW_BYTES + NOALLOC_STATS_BYTES);
        spec_and_normalise(s, mix, b, L, 4096, frame_buf, xspec, xwave, norms, stats, twiddles);
    });
}

int dmx_op_ispec_sum(void *stream, const float *xspec, const float *xtime, int b, int L, const float *norms,
                     float *stems) {
    return guarded([&] {
        hipStream_t s = as_stream(stream);
        int le = (L + 1023) / 1024, rows = b * 8;
        Scratch scratch(((size_t)rows * le * 4096 + (size_t)rows * le * 2048 * 2) * sizeof(float));
        ispec_and_sum(s, xspec, xtime, b, 4, L, 4096, le, norms, static_cast<float *>(scratch.p), stems,
                      twiddles_4096());
        DMX_HIP(hipStreamSynchronize(s));
    });
}

}  // extern "C"
