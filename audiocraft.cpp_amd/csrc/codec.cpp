// codec.cpp -- the EnCodec / SEANet decoder of include/mgx.h on the GPU: RVQ codes -> audio.
//
// Reference: rvq_decode (src/mg/encodec.h:69-84) and codec_decode (src/ac/codec.h:127-146) over
// seanet_decode_pre / lstm_graph / seanet_decode_post (src/ac/seanet.h:282-317, src/ac/lstm.h:
// 44-101), as MusicGen's 32 kHz EnCodec configures them (ELU, ratios [8, 5, 4, 4], 2-layer LSTM,
// 4 x 2048 codebooks). The codebooks and every weight stay resident; a decode is the lookup, the
// input conv, the LSTM (input projection as one 1 x 1 convolution over every frame, then one
// launch per step), the four upsampling stages (ELU, transposed conv, residual block) and the
// output conv, all f32.
#include "codec_kernels.h"
#include "host.h"

#include <memory>
#include <mutex>

using namespace mgxh;

struct mgx_codec {
    mgx_codec_config c{};
    int device = 0;
    DevArena mem;
    hipStream_t hs = nullptr;
    std::mutex mu;   // one decode at a time: the working buffers are shared
    struct Conv {
        const float *w = nullptr, *b = nullptr;
        int cin = 0, cout = 0, k = 0;
    };
    struct Lstm {
        Conv ih;                     // w_ih as a 1 x 1 convolution, bias fused
        const float* w_hh = nullptr;
    };
    struct Res {
        Conv c1, c2;
        int dil = 1;
    };
    struct Stage {
        const float *wt = nullptr, *bt = nullptr;
        int cin = 0, cout = 0, k = 0, ratio = 1;
        std::vector<Res> res;
    };
    const float* embed = nullptr;    // [n_q][bins][latent_dim]
    Conv in, out;
    std::vector<Lstm> lstm;
    std::vector<Stage> stages;
    int bott = 0;                    // bottleneck channels
    // working buffers, grown to the longest decode so far
    DevArena work;
    size_t cap_frames = 0;
    int32_t* codes = nullptr;
    float *latent = nullptr, *x0 = nullptr, *proj = nullptr, *hst = nullptr, *cst = nullptr;
    float *buf[3] = {};
    ~mgx_codec() {
        if (hs) (void)hipStreamSynchronize(hs);
        work.release();
        mem.release();
        if (hs) (void)hipStreamDestroy(hs);
    }
};

namespace {

const float* need_f32(DevArena& mem, const mgx_tensor* t, int n, const std::string& name,
                      std::initializer_list<int64_t> ne, hipStream_t s) {
    const mgx_tensor* x = find(t, n, name);
    if (!x) throw Error(MGX_ERR_INVALID, "missing tensor " + name);
    if (x->type != mgx::T_F32 || !x->data) throw Error(MGX_ERR_INVALID, name + " must be f32");
    size_t count = 1;
    int d = 0;
    for (int64_t v : ne) {
        if (x->ne[d] != v) throw Error(MGX_ERR_INVALID, "bad shape for " + name);
        count *= (size_t)v;
        ++d;
    }
    for (; d < 4; ++d)
        if (x->ne[d] > 1) throw Error(MGX_ERR_INVALID, "bad shape for " + name);
    if (x->nbytes && x->nbytes < count * 4) throw Error(MGX_ERR_INVALID, "short data for " + name);
    float* p = mem.alloc<float>(count);
    HIP_OK(hipMemcpyAsync(p, x->data, count * 4, hipMemcpyHostToDevice, s));
    return p;
}

mgx_codec::Conv load_conv(mgx_codec* m, const mgx_tensor* t, int n, const std::string& p, int cin, int cout, int k) {
    mgx_codec::Conv c;
    c.cin = cin; c.cout = cout; c.k = k;
    c.w = need_f32(m->mem, t, n, p + ".weight", {k, cin, cout}, m->hs);   // ggml [k, in, out]
    c.b = need_f32(m->mem, t, n, p + ".bias", {cout}, m->hs);
    return c;
}

void codec_create(const mgx_codec_config* cfg, const mgx_tensor* t, int n, mgx_codec** out) {
    if (!cfg || !t || !out) throw Error(MGX_ERR_INVALID, "null argument");
    *out = nullptr;
    const mgx_codec_config& c = *cfg;
    if (!c.elu) throw Error(MGX_ERR_INVALID, "only ELU codecs (MusicGen's EnCodec) are supported");
    if (c.n_ratios <= 0 || c.n_ratios > 8) throw Error(MGX_ERR_INVALID, "codec has no ratios");
    int hop = 1;
    for (int i = 0; i < c.n_ratios; ++i) {
        if (c.ratios[i] <= 0) throw Error(MGX_ERR_INVALID, "bad codec ratio");
        hop *= c.ratios[i];
    }
    if (hop != c.hop_length) throw Error(MGX_ERR_INVALID, "codec ratio product disagrees with the declared hop length");
    if (c.channels <= 0 || c.n_filters <= 0 || c.latent_dim <= 0 || c.kernel_size <= 0 || c.last_kernel_size <= 0 ||
        c.residual_kernel_size <= 0 || c.compress <= 0 || c.lstm_layers < 0 || c.n_residual_layers < 0 ||
        c.dilation_base <= 0)
        throw Error(MGX_ERR_INVALID, "bad codec config");
    if (c.rvq && (c.rvq_n_q <= 0 || c.rvq_bins <= 0)) throw Error(MGX_ERR_INVALID, "bad RVQ config");
    auto m = std::make_unique<mgx_codec>();
    m->c = c;
    HIP_OK(hipGetDevice(&m->device));
    HIP_OK(hipStreamCreateWithFlags(&m->hs, hipStreamNonBlocking));
    hipStream_t s = m->hs;
    int mult = 1 << c.n_ratios;
    m->bott = c.n_filters * mult;
    if (c.rvq) {
        float* e = m->mem.alloc<float>((size_t)c.rvq_n_q * c.rvq_bins * c.latent_dim);
        for (int l = 0; l < c.rvq_n_q; ++l) {
            const std::string name = "codec.rvq." + std::to_string(l) + ".embed";
            const mgx_tensor* x = find(t, n, name);
            if (!x) throw Error(MGX_ERR_INVALID, "missing tensor " + name);
            if (x->type != mgx::T_F32 || x->ne[0] != c.latent_dim || x->ne[1] != c.rvq_bins || !x->data)
                throw Error(MGX_ERR_INVALID, "codebook " + std::to_string(l) + " is not [dim, bins] f32");
            HIP_OK(hipMemcpyAsync(e + (size_t)l * c.rvq_bins * c.latent_dim, x->data,
                                  sizeof(float) * (size_t)c.rvq_bins * c.latent_dim, hipMemcpyHostToDevice, s));
        }
        m->embed = e;
    }
    m->in = load_conv(m.get(), t, n, "codec.decoder.in", c.latent_dim, m->bott, c.kernel_size);
    for (int l = 0; l < c.lstm_layers; ++l) {
        const std::string p = "codec.decoder.lstm." + std::to_string(l) + ".";
        mgx_codec::Lstm ly;
        ly.ih.cin = m->bott; ly.ih.cout = 4 * m->bott; ly.ih.k = 1;
        ly.ih.w = need_f32(m->mem, t, n, p + "w_ih", {m->bott, 4 * m->bott}, s);
        ly.ih.b = need_f32(m->mem, t, n, p + "bias", {4 * m->bott}, s);
        ly.w_hh = need_f32(m->mem, t, n, p + "w_hh", {m->bott, 4 * m->bott}, s);
        m->lstm.push_back(ly);
    }
    for (int st = 0; st < c.n_ratios; ++st) {
        const std::string p = "codec.decoder.stage." + std::to_string(st) + ".";
        mgx_codec::Stage sg;
        sg.ratio = c.ratios[st];
        sg.cin = c.n_filters * mult;
        sg.cout = sg.cin / 2;
        sg.k = 2 * sg.ratio;
        // ggml [in, kernel * out]: row o * kernel + j holds the in-channel weights
        sg.wt = need_f32(m->mem, t, n, p + "up.weight_col2im", {sg.cin, (int64_t)sg.k * sg.cout}, s);
        sg.bt = need_f32(m->mem, t, n, p + "up.bias", {sg.cout}, s);
        for (int j = 0; j < c.n_residual_layers; ++j) {
            mgx_codec::Res r;
            for (int d = 0; d < j; ++d) r.dil *= c.dilation_base;
            const int hid = sg.cout / c.compress;
            const std::string rp = p + "res." + std::to_string(j) + ".";
            r.c1 = load_conv(m.get(), t, n, rp + "conv1", sg.cout, hid, c.residual_kernel_size);
            r.c2 = load_conv(m.get(), t, n, rp + "conv2", hid, sg.cout, 1);
            sg.res.push_back(r);
        }
        m->stages.push_back(sg);
        mult /= 2;
    }
    m->out = load_conv(m.get(), t, n, "codec.decoder.out", c.n_filters, c.channels, c.last_kernel_size);
    HIP_OK(hipGetLastError());
    HIP_OK(hipStreamSynchronize(s));
    *out = m.release();
}

void conv(mgx_codec* m, const mgx_codec::Conv& cv, const float* x, int T, int dil, bool elu, const float* skip,
          float* y) {
    const int total = (cv.k - 1) * dil, right = total / 2, left = total - right;
    if (T <= (left > right ? left : right))
        throw Error(MGX_ERR_INVALID, "input of " + std::to_string(T) + " frames is too short for the codec's convolutions");
    mgx::ConvArgs a{};
    a.x = x; a.cin = cv.cin; a.T = T; a.w = cv.w; a.b = cv.b; a.cout = cv.cout; a.k = cv.k; a.dil = dil;
    a.pad_left = left; a.elu = elu ? 1 : 0; a.skip = skip; a.y = y;
    mgx::launch_conv1d(a, m->hs);
}

// Working buffers for `frames` latent frames: the largest feature map is a stage's channels
// times its length, at most n_filters * 2 * hop * frames (the last stage, and bott * frames).
void reserve(mgx_codec* m, size_t frames) {
    if (frames <= m->cap_frames) return;
    HIP_OK(hipStreamSynchronize(m->hs));
    m->work.release();
    const mgx_codec_config& c = m->c;
    size_t big = (size_t)m->bott * frames;
    size_t len = frames;
    for (const auto& sg : m->stages) {
        len *= (size_t)sg.ratio;
        big = std::max(big, (size_t)sg.cin * len);   // cout * len and the residual hidden fit too
    }
    big = std::max(big, (size_t)c.channels * len);
    m->codes = m->work.alloc<int32_t>((size_t)std::max(c.rvq_n_q, 1) * frames);
    m->latent = m->work.alloc<float>((size_t)c.latent_dim * frames);
    m->x0 = m->work.alloc<float>((size_t)m->bott * frames);
    m->proj = m->work.alloc<float>((size_t)4 * m->bott * frames);
    m->hst = m->work.alloc<float>((size_t)2 * m->bott);
    m->cst = m->work.alloc<float>((size_t)m->bott);
    for (auto& b : m->buf) b = m->work.alloc<float>(big);
    m->cap_frames = frames;
}

// latent (device, [latent_dim][frames]) -> audio_out (host, [channels][frames * hop])
void decode_latent(mgx_codec* m, const float* latent, int frames, float* audio_out) {
    const mgx_codec_config& c = m->c;
    hipStream_t s = m->hs;
    const int B = m->bott;
    // decoder.in (seanet_decode_pre)
    conv(m, m->in, latent, frames, 1, false, nullptr, m->x0);
    // StreamableLSTM: every layer's input projection at once, then the recurrence; the last
    // layer adds the skip from the LSTM's input
    const float* input = m->x0;
    float* layer_out = m->buf[0];
    for (size_t l = 0; l < m->lstm.size(); ++l) {
        conv(m, m->lstm[l].ih, input, frames, 1, false, nullptr, m->proj);
        HIP_OK(hipMemsetAsync(m->hst, 0, sizeof(float) * 2 * B, s));
        HIP_OK(hipMemsetAsync(m->cst, 0, sizeof(float) * B, s));
        const bool last = l + 1 == m->lstm.size();
        for (int t = 0; t < frames; ++t) {
            mgx::LstmStepArgs a{};
            a.w_hh = m->lstm[l].w_hh; a.proj = m->proj; a.H = B; a.T = frames; a.t = t;
            a.h_prev = m->hst + (size_t)(t & 1) * B;
            a.h_next = m->hst + (size_t)((t + 1) & 1) * B;
            a.c = m->cst; a.out = layer_out; a.skip = last ? m->x0 : nullptr;
            mgx::launch_lstm_step(a, s);
        }
        input = layer_out;
        layer_out = layer_out == m->buf[0] ? m->buf[1] : m->buf[0];
    }
    // stages (seanet_decode_post): x, then h (residual hidden), then the sum
    const float* x = m->lstm.empty() ? m->x0 : input;
    int T = frames;
    float* pool[3] = {m->buf[0], m->buf[1], m->buf[2]};
    auto other = [&](const float* a, const float* b) {
        for (float* p : pool)
            if (p != a && p != b) return p;
        return pool[0];
    };
    for (const auto& sg : m->stages) {
        float* up = other(x, nullptr);
        mgx::ConvTArgs a{};
        a.x = x; a.cin = sg.cin; a.T = T; a.w = sg.wt; a.b = sg.bt; a.cout = sg.cout; a.k = sg.k; a.stride = sg.ratio;
        a.pad_left = (sg.k - sg.ratio) - (sg.k - sg.ratio) / 2; a.elu = 1; a.y = up;
        mgx::launch_conv_transpose1d(a, s);
        T *= sg.ratio;
        x = up;
        for (const auto& r : sg.res) {
            float* h = other(x, nullptr);
            conv(m, r.c1, x, T, r.dil, true, nullptr, h);
            float* y = other(x, h);
            conv(m, r.c2, h, T, 1, true, x, y);
            x = y;
        }
    }
    float* audio = other(x, nullptr);
    conv(m, m->out, x, T, 1, true, nullptr, audio);
    HIP_OK(hipGetLastError());
    HIP_OK(hipMemcpyAsync(audio_out, audio, sizeof(float) * (size_t)c.channels * T, hipMemcpyDeviceToHost, s));
    HIP_OK(hipStreamSynchronize(s));
}

}  // namespace

extern "C" {

int mgx_codec_create(const mgx_codec_config* config, const mgx_tensor* tensors, int32_t n, mgx_codec** out) {
    return guarded([&] { codec_create(config, tensors, n, out); });
}

int mgx_codec_decode(mgx_codec* m, const int32_t* codes, int32_t frames, float* audio_out) {
    return guarded([&] {
        if (!m || !codes || !audio_out) throw Error(MGX_ERR_INVALID, "null argument");
        const mgx_codec_config& c = m->c;
        if (!c.rvq) throw Error(MGX_ERR_INVALID, "the codec has no residual quantizer");
        if (frames <= 0) throw Error(MGX_ERR_INVALID, "codes do not hold n_q * frames values");
        for (int64_t i = 0; i < (int64_t)c.rvq_n_q * frames; ++i)
            if (codes[i] < 0 || codes[i] >= c.rvq_bins) throw Error(MGX_ERR_INVALID, "a code is outside [0, bins)");
        std::lock_guard<std::mutex> lk(m->mu);
        HIP_OK(hipSetDevice(m->device));
        reserve(m, (size_t)frames);
        HIP_OK(hipMemcpyAsync(m->codes, codes, sizeof(int32_t) * (size_t)c.rvq_n_q * frames, hipMemcpyHostToDevice,
                              m->hs));
        mgx::launch_rvq_decode(m->embed, m->codes, c.rvq_n_q, c.rvq_bins, c.latent_dim, frames, m->latent, m->hs);
        decode_latent(m, m->latent, frames, audio_out);
    });
}

int mgx_codec_decode_latent(mgx_codec* m, const float* latent, int32_t frames, float* audio_out) {
    return guarded([&] {
        if (!m || !latent || !audio_out) throw Error(MGX_ERR_INVALID, "null argument");
        if (frames <= 0) throw Error(MGX_ERR_INVALID, "latent does not hold frames * latent_dim values");
        std::lock_guard<std::mutex> lk(m->mu);
        HIP_OK(hipSetDevice(m->device));
        reserve(m, (size_t)frames);
        HIP_OK(hipMemcpyAsync(m->latent, latent, sizeof(float) * (size_t)m->c.latent_dim * frames,
                              hipMemcpyHostToDevice, m->hs));
        decode_latent(m, m->latent, frames, audio_out);
    });
}

void mgx_codec_destroy(mgx_codec* m) { delete m; }

}  // extern "C"
