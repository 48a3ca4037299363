// t5.cpp -- the T5-base text encoder of include/mgx.h on the GPU.
//
// Reference: ac::T5EncoderConfig and ac::t5_encode (src/ac/t5.h:20-140) as ac::encode_prompt
// runs them (src/ac/conditioner.h:56-108): one prompt, its own token count, no padding. The
// reference loads the encoder from its GGUF and frees it inside every call; here the encoder
// stays resident (0.2 GB at F16 against 288 GB of HBM) and an encode is only the forward.
//
// Per layer: RMS norm -> q and k|v projections (f32 source, the GEMV's own activation
// conversion) -> attention of every query over all keys with the learned relative-position
// bias added to the unscaled q.k score (the cross-attention kernel with a bias row and shared
// keys) -> o projection added to the residual; RMS norm -> wi -> ReLU (into wo's activation
// form) -> wo added to the residual. Final RMS norm. Every reduction has the oracle's fixed
// order, so the output equals the oracle's bit for bit.
#include "host.h"

#include <cmath>
#include <memory>
#include <mutex>

using namespace mgxh;

// The working memory of mgx_t5_encode_static (see there).
constexpr size_t T5_STATIC_BYTES = (size_t)32 << 20;
static __device__ __align__(256) uint8_t scratch[T5_STATIC_BYTES];

namespace {

constexpr int T5_MAX_TOKENS = 256;   // the attention kernels' key bound; ac.t5.max_length is 256
constexpr int T5_REL = 2 * T5_MAX_TOKENS - 1;   // relative positions key - query in [-255, 255]

// An activation buffer in the form a weight type's GEMV reads, for `cols` columns of `n`.
mgx::ActBuf act_buf(DevArena& mem, int wtype, int cols, int n) {
    mgx::ActBuf a{};
    a.stride = n;
    if (wtype == mgx::T_Q8_0 || wtype == mgx::T_Q4_0) {
        a.kind = mgx::ACT_Q8;
        a.q = mem.alloc<int8_t>((size_t)cols * n);
        a.d = mem.alloc<float>((size_t)cols * n / 32);
    } else if (wtype == mgx::T_F16) {
        a.kind = mgx::ACT_F16;
        a.h = mem.alloc<uint16_t>((size_t)cols * n);
    } else {
        a.kind = mgx::ACT_F32;
        a.f = mem.alloc<float>((size_t)cols * n);
    }
    return a;
}

}  // namespace

struct mgx_t5 {
    mgx_t5_config c{};
    int device = 0;
    DevArena mem;
    hipStream_t hs = nullptr;
    std::mutex mu;   // one encode at a time: the working buffers are shared
    mgx::DevMat emb{}, rel{};
    struct Layer {
        mgx::DevMat q, kv, o, wi, wo;
        const float *an, *fn;
        mgx::ActBuf att, ff;   // o's and wo's activation forms
    };
    std::vector<Layer> L;
    const float* fnorm = nullptr;
    int32_t *ids = nullptr, *relb = nullptr;
    float *x = nullptr, *h = nullptr, *q = nullptr, *kvp = nullptr, *k = nullptr, *v = nullptr, *f = nullptr;
    float* bias = nullptr;
    ~mgx_t5() {
        if (hs) (void)hipStreamSynchronize(hs);
        mem.release();
        if (hs) (void)hipStreamDestroy(hs);
    }
};

namespace {

void t5_create(const mgx_t5_config* cfg, const mgx_tensor* t, int n, mgx_t5** out) {
    if (!cfg || !t || !out) throw Error(MGX_ERR_INVALID, "null argument");
    *out = nullptr;
    const mgx_t5_config& c = *cfg;
    if (c.dim <= 0 || c.layers <= 0 || c.heads <= 0 || c.intermediate <= 0 || c.vocab <= 0 ||
        c.relative_buckets < 2 || c.relative_max_distance <= 0 || !(c.eps >= 0.0f))
        throw Error(MGX_ERR_INVALID, "bad T5 config");
    if (c.head_dim != 64) throw Error(MGX_ERR_INVALID, "T5 head_dim must be 64");
    if (c.dim % 32 || c.intermediate % 32 || c.dim > 2048)
        throw Error(MGX_ERR_INVALID, "T5 widths must be multiples of 32 (dim at most 2048)");
    const int D = c.dim, inner = c.heads * 64, F = c.intermediate;
    auto m = std::make_unique<mgx_t5>();
    m->c = c;
    HIP_OK(hipGetDevice(&m->device));
    HIP_OK(hipStreamCreateWithFlags(&m->hs, hipStreamNonBlocking));
    hipStream_t s = m->hs;
    m->emb = load_mat(m->mem, t, n, "te.embed.weight", D, c.vocab, s);
    m->rel = load_mat(m->mem, t, n, "te.relative_attention_bias.weight", c.heads, c.relative_buckets, s);
    if (m->rel.type != mgx::T_F32 && m->rel.type != mgx::T_F16)
        throw Error(MGX_ERR_INVALID, "te.relative_attention_bias.weight must be F32 or F16");
    m->fnorm = load_vec(m->mem, t, n, "te.norm.weight", D, s);
    for (int l = 0; l < c.layers; ++l) {
        const std::string p = "te." + std::to_string(l) + ".";
        mgx_t5::Layer ly{};
        ly.an = load_vec(m->mem, t, n, p + "attn_norm.weight", D, s);
        ly.fn = load_vec(m->mem, t, n, p + "ffn_norm.weight", D, s);
        ly.q = load_mat(m->mem, t, n, p + "q.weight", D, inner, s);
        // k and v as one [2 * inner][dim] matrix: one GEMV launch, the same rows
        const mgx_tensor& tk = need(t, n, p + "k.weight", D, inner);
        const mgx_tensor& tv = need(t, n, p + "v.weight", D, inner);
        if (tk.type != tv.type) throw Error(MGX_ERR_INVALID, p + "k.weight and " + p + "v.weight differ in type");
        ly.kv = alloc_mat(m->mem, tk.type, D, 2 * inner);
        upload_rows(tk, ly.kv, 0, s);
        upload_rows(tv, ly.kv, inner, s);
        ly.o = load_mat(m->mem, t, n, p + "o.weight", inner, D, s);
        ly.wi = load_mat(m->mem, t, n, p + "wi.weight", D, F, s);
        ly.wo = load_mat(m->mem, t, n, p + "wo.weight", F, D, s);
        ly.att = act_buf(m->mem, ly.o.type, T5_MAX_TOKENS, inner);
        ly.ff = act_buf(m->mem, ly.wo.type, T5_MAX_TOKENS, F);
        m->L.push_back(ly);
    }
    const size_t N = T5_MAX_TOKENS;
    m->ids = m->mem.alloc<int32_t>(N);
    m->relb = m->mem.alloc<int32_t>(T5_REL);
    m->x = m->mem.alloc<float>(N * D);
    m->h = m->mem.alloc<float>(N * D);
    m->q = m->mem.alloc<float>(N * inner);
    m->kvp = m->mem.alloc<float>(N * 2 * inner);
    m->k = m->mem.alloc<float>(N * inner);
    m->v = m->mem.alloc<float>(N * inner);
    m->f = m->mem.alloc<float>(N * F);
    m->bias = m->mem.alloc<float>((size_t)c.heads * N * N);
    HIP_OK(hipGetLastError());
    HIP_OK(hipStreamSynchronize(s));
    *out = m.release();
}

// The working buffers of one encode: the encoder's own (mgx_t5_encode) or carved from the
// static scratch array (mgx_t5_encode_static). att / ff: byte regions holding each layer's o and
// wo activation form (null: the encoder's per-layer buffers).
struct T5Work {
    int32_t *ids, *rel;
    float *x, *h, *q, *kvp, *k, *v, *f, *bias;
    uint8_t *att, *ff;
};

// An activation form of `cols` columns of `n` aliased onto a byte region of 4 * cols * n bytes
// (enough for any form: Q8 needs n + n / 8 bytes per column, F16 2n, F32 4n).
mgx::ActBuf act_in(uint8_t* region, int wtype, int cols, int n) {
    mgx::ActBuf a{};
    a.stride = n;
    if (wtype == mgx::T_Q8_0 || wtype == mgx::T_Q4_0) {
        a.kind = mgx::ACT_Q8;
        a.q = (int8_t*)region;
        a.d = (float*)(region + ((size_t)cols * n + 255) / 256 * 256);
    } else if (wtype == mgx::T_F16) {
        a.kind = mgx::ACT_F16;
        a.h = (uint16_t*)region;
    } else {
        a.kind = mgx::ACT_F32;
        a.f = (float*)region;
    }
    return a;
}

// Argument checks of an encode (before any device work).
void check_ids(const mgx_t5* m, const int32_t* ids, int seq, const float* out) {
    if (!m || !ids || !out) throw Error(MGX_ERR_INVALID, "null argument");
    if (seq <= 0 || seq > T5_MAX_TOKENS) throw Error(MGX_ERR_INVALID, "a T5 prompt holds 1 to 256 tokens");
    for (int i = 0; i < seq; ++i)
        if (ids[i] < 0 || ids[i] >= m->c.vocab) throw Error(MGX_ERR_INVALID, "token id out of range");
}

// The relative-position buckets of key - query = r - 255 for r in [0, 511) (t5.h:46-76), into
// a caller buffer of T5_REL ints.
void rel_buckets(const mgx_t5_config& c, int32_t* out) {
    for (int r = 0; r < T5_REL; ++r)
        out[r] = mgx_t5_relative_bucket(r - (T5_MAX_TOKENS - 1), c.relative_buckets, c.relative_max_distance);
}

// The forward: embeddings, the layers, the final norm into w.h; the ids and the relative
// buckets are already in w.ids / w.rel. Launches on s, no synchronization.
void encode_body(mgx_t5* m, const T5Work& w, int seq, hipStream_t s) {
    const mgx_t5_config& c = m->c;
    const int D = c.dim, H = c.heads, inner = H * 64, F = c.intermediate;
    mgx::launch_rows(m->emb, w.ids, seq, w.x, s);
    mgx::launch_t5_bias(m->rel, w.rel, T5_MAX_TOKENS - 1, seq, H, w.bias, s);
    for (const mgx_t5::Layer& ly : m->L) {
        const mgx::ActBuf att = w.att ? act_in(w.att, ly.o.type, seq, inner) : ly.att;
        const mgx::ActBuf ff = w.ff ? act_in(w.ff, ly.wo.type, seq, F) : ly.ff;
        mgx::launch_rms(w.x, D, seq, D, ly.an, c.eps, w.h, s);
        mgx::GemvArgs a = ga(ly.q, seq);
        mgx::launch_gemv(epi_store(pro_f32(a, w.h, D), w.q, inner), s);
        mgx::GemvArgs b = ga(ly.kv, seq);
        mgx::launch_gemv(epi_store(pro_f32(b, w.h, D), w.kvp, 2 * inner), s);
        mgx::launch_xkv_split(w.kvp, seq, seq, inner, w.k, w.v, s);
        mgx::XAttnArgs xa{};
        xa.q = w.q; xa.k = w.k; xa.v = w.v; xa.n_ctx = seq; xa.dim = inner; xa.scale = 1.0f;
        xa.out = att;
        xa.bias = w.bias; xa.bias_stride = seq; xa.shared_kv = 1;
        mgx::launch_xattn(xa, H, seq, s);
        mgx::GemvArgs o = ga(ly.o, seq);
        mgx::launch_gemv(epi_store(pro_act(o, att), w.x, D, true), s);
        mgx::launch_rms(w.x, D, seq, D, ly.fn, c.eps, w.h, s);
        mgx::GemvArgs wi = ga(ly.wi, seq);
        mgx::launch_gemv(epi_store(pro_f32(wi, w.h, D), w.f, F), s);
        mgx::launch_relu_act(w.f, F, seq, ff, s);
        mgx::GemvArgs wo = ga(ly.wo, seq);
        mgx::launch_gemv(epi_store(pro_act(wo, ff), w.x, D, true), s);
    }
    mgx::launch_rms(w.x, D, seq, D, m->fnorm, c.eps, w.h, s);
    HIP_OK(hipGetLastError());
}

void t5_encode(mgx_t5* m, const int32_t* ids, int seq, float* out) {
    check_ids(m, ids, seq, out);
    const mgx_t5_config& c = m->c;
    std::lock_guard<std::mutex> lk(m->mu);
    HIP_OK(hipSetDevice(m->device));
    hipStream_t s = m->hs;
    std::vector<int32_t> rel(T5_REL);
    rel_buckets(c, rel.data());
    HIP_OK(hipMemcpyAsync(m->ids, ids, sizeof(int32_t) * seq, hipMemcpyHostToDevice, s));
    HIP_OK(hipMemcpyAsync(m->relb, rel.data(), sizeof(int32_t) * T5_REL, hipMemcpyHostToDevice, s));
    const T5Work w{m->ids, m->relb, m->x, m->h, m->q, m->kvp, m->k, m->v, m->f, m->bias, nullptr, nullptr};
    encode_body(m, w, seq, s);
    HIP_OK(hipMemcpyAsync(out, m->h, sizeof(float) * (size_t)seq * c.dim, hipMemcpyDeviceToHost, s));
    HIP_OK(hipStreamSynchronize(s));
}

// ------------------------------------------------------------------------------------
// mgx_t5_encode_static: the same encode with every working buffer in `scratch`, a file-scope
// device array of T5_STATIC_BYTES. Each device the call runs on holds its own copy for the
// life of the process; the call allocates nothing. Its address on a device is looked up once
// (hipGetSymbolAddress with that device current) and kept per device; host code uses that
// address, never the array's name. Calls share the array: two that overlap on one device race.
// ------------------------------------------------------------------------------------
constexpr int T5_MAX_DEVICES = 64;

std::mutex g_scratch_mu;
uint8_t* g_scratch[T5_MAX_DEVICES] = {};

// The scratch array's address on `device` (which must be current).
uint8_t* scratch_on(int device) {
    if (device < 0 || device >= T5_MAX_DEVICES) throw Error(MGX_ERR_DEVICE, "device ordinal out of range");
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch[device]) {
        void* p = nullptr;
        const hipError_t rc = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (rc != hipSuccess || !p)
            throw Error(MGX_ERR_DEVICE, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(rc));
        g_scratch[device] = (uint8_t*)p;
    }
    return g_scratch[device];
}

// The working buffers of an encode of seq tokens carved from base (256-byte aligned pieces);
// returns the bytes used.
size_t carve(const mgx_t5_config& c, int seq, uint8_t* base, T5Work* w) {
    const size_t D = c.dim, inner = (size_t)c.heads * 64, F = c.intermediate, n = seq;
    size_t off = 0;
    auto take = [&](size_t bytes) { uint8_t* p = base ? base + off : nullptr; off += (bytes + 255) / 256 * 256; return p; };
    w->ids = (int32_t*)take(4 * n);
    w->rel = (int32_t*)take(4 * (size_t)T5_REL);
    w->x = (float*)take(4 * n * D);
    w->h = (float*)take(4 * n * D);
    w->q = (float*)take(4 * n * inner);
    w->kvp = (float*)take(8 * n * inner);
    w->k = (float*)take(4 * n * inner);
    w->v = (float*)take(4 * n * inner);
    w->f = (float*)take(4 * n * F);
    w->bias = (float*)take(4 * (size_t)c.heads * n * n);
    w->att = take(4 * n * inner + 256);
    w->ff = take(4 * n * F + 256);
    return off;
}

void t5_encode_static(mgx_t5* m, const int32_t* ids, int seq, float* out) {
    check_ids(m, ids, seq, out);
    const mgx_t5_config& c = m->c;
    T5Work w{};
    const size_t need = carve(c, seq, nullptr, &w);
    if (need > T5_STATIC_BYTES)
        throw Error(MGX_ERR_INVALID, "this encode needs " + std::to_string(need >> 20) + " MiB of scratch; the static "
                                     "scratch holds " + std::to_string(T5_STATIC_BYTES >> 20) + " MiB (use mgx_t5_encode)");
    std::lock_guard<std::mutex> lk(m->mu);
    HIP_OK(hipSetDevice(m->device));
    uint8_t* base = scratch_on(m->device);
    carve(c, seq, base, &w);
    int32_t rel[T5_REL];
    rel_buckets(c, rel);
    hipStream_t s = m->hs;
    HIP_OK(hipMemcpyAsync(w.ids, ids, sizeof(int32_t) * seq, hipMemcpyHostToDevice, s));
    HIP_OK(hipMemcpyAsync(w.rel, rel, sizeof(rel), hipMemcpyHostToDevice, s));
    encode_body(m, w, seq, s);
    HIP_OK(hipMemcpyAsync(out, w.h, sizeof(float) * (size_t)seq * c.dim, hipMemcpyDeviceToHost, s));
    HIP_OK(hipStreamSynchronize(s));
}

}  // namespace

extern "C" {

// transformers' T5Attention._relative_position_bucket, bidirectional (t5.h:46-61): the upper
// half of the buckets holds keys after the query; distances below a quarter of the buckets map
// one to one, longer ones logarithmically (f32 logarithms) up to max_distance.
int32_t mgx_t5_relative_bucket(int32_t relative_position, int32_t num_buckets, int32_t max_distance) {
    const int half = num_buckets / 2, exact = half / 2;
    const int base = relative_position > 0 ? half : 0;
    const int dist = relative_position < 0 ? -relative_position : relative_position;
    if (dist < exact) return base + dist;
    int far = exact;
    const float span = std::log((float)max_distance / (float)exact);
    if (span > 0.0f) far += (int)(std::log((float)dist / (float)exact) / span * (float)(half - exact));
    return base + (far < half - 1 ? far : half - 1);
}

int mgx_t5_create(const mgx_t5_config* config, const mgx_tensor* tensors, int32_t n, mgx_t5** out) {
    return guarded([&] { t5_create(config, tensors, n, out); });
}

int mgx_t5_encode(mgx_t5* t5, const int32_t* ids, int32_t n_tokens, float* hidden_out) {
    return guarded([&] { t5_encode(t5, ids, n_tokens, hidden_out); });
}

int mgx_t5_encode_static(mgx_t5* t5, const int32_t* ids, int32_t n_tokens, float* hidden_out) {
    return guarded([&] { t5_encode_static(t5, ids, n_tokens, hidden_out); });
}

void mgx_t5_destroy(mgx_t5* t5) { delete t5; }

}  // extern "C"
