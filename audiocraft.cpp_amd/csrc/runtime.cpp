// runtime.cpp -- the C ABI of include/mgx.h: weights, streams (Decoder), forward and the
// generation loop, all driving the kernels of kernels.hip on one HIP stream.
//
// Reference counterparts: GgufModel / load_gguf (src/gguf_model.h:241-414), LmConfig::from
// (src/mg/lm.h:60-90), Decoder (src/mg/pipeline.cpp:36-195), mg_generate (pipeline.cpp:
// 199-314), KvCache (src/mg/kv_cache.h:33-115), Rng (src/rng.h:15-33), DelayPattern
// (src/mg/pattern.h:31-115).
#include "mgx.h"
#include "kernels.h"

#include <hip/hip_runtime.h>

#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <algorithm>
#include <map>
#include <memory>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

thread_local std::string g_error;

struct Error : std::runtime_error {
    int code;
    Error(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

#define HIP_OK(expr)                                                                            \
    do {                                                                                        \
        hipError_t e_ = (expr);                                                                 \
        if (e_ != hipSuccess)                                                                   \
            throw Error(MGX_ERR_DEVICE, std::string(#expr) + ": " + hipGetErrorString(e_));     \
    } while (0)

template <typename F> int guarded(F&& f) {
    try {
        f();
        return MGX_OK;
    } catch (const Error& e) {
        g_error = e.what();
        return e.code;
    } catch (const std::exception& e) {
        g_error = e.what();
        return MGX_ERR_INVALID;
    }
}

double now_s() {
    using clock = std::chrono::steady_clock;
    return std::chrono::duration<double>(clock::now().time_since_epoch()).count();
}

// Device allocations owned by one object, freed together.
struct DevArena {
    std::vector<void*> ptrs;
    template <typename T> T* alloc(size_t count) {
        void* p = nullptr;
        if (count == 0) count = 1;
        HIP_OK(hipMalloc(&p, count * sizeof(T)));
        ptrs.push_back(p);
        return (T*)p;
    }
    void release() {
        for (void* p : ptrs) (void)hipFree(p);
        ptrs.clear();
    }
};

enum { P_QKV, P_OUT, P_CQ, P_CKV, P_COUT, P_FF0, P_FF2, P_COUNT };
const char* const PROJ[P_COUNT] = {"self.qkv", "self.out", "cross.q", "cross.kv", "cross.out", "ff.0", "ff.2"};

int act_kind(int wtype) {
    return (wtype == mgx::T_Q8_0 || wtype == mgx::T_Q4_0) ? mgx::ACT_Q8 : (wtype == mgx::T_F16 ? mgx::ACT_F16 : mgx::ACT_F32);
}

}  // namespace

struct LayerW {
    mgx::DevMat w[P_COUNT];
    const float *n1w, *n1b, *ncw, *ncb, *n2w, *n2b;
};

struct mgx_model {
    mgx_lm_config c{};
    int device = 0;
    DevArena mem;
    mgx::DevMat emb[8]{}, heads{}, cond_proj{};
    const float *cond_proj_b = nullptr, *out_w = nullptr, *out_b = nullptr;
    std::vector<LayerW> L;
    ~mgx_model() { mem.release(); }
};

struct mgx_stream {
    mgx_model* m = nullptr;
    int cap = 0, n_seq = 0, cross = 0, n_ctx = 0, used = 0, forwards = 0, max_chunks = 0, max_in = 0;
    hipStream_t hs = nullptr;
    DevArena mem;
    float *K = nullptr, *V = nullptr;        // per layer [n_seq][H][cap][64]
    float *xk = nullptr, *xv = nullptr;      // per layer [H][n_ctx][64], stream 0
    float* pos = nullptr;                    // [cap][dim]
    float *x = nullptr, *qb = nullptr, *ff = nullptr, *scores = nullptr, *opart = nullptr, *logits = nullptr;
    float *qc = nullptr, *oc = nullptr;      // cross q, cross attention output [dim]
    int8_t* aq = nullptr;
    float* ad = nullptr;
    uint16_t* ah = nullptr;
    float* af = nullptr;
    int32_t* ids = nullptr;                  // [n_q][cap] staged ids for mgx_forward
    ~mgx_stream() {
        if (hs) (void)hipStreamSynchronize(hs);
        mem.release();
        if (hs) (void)hipStreamDestroy(hs);
    }
    mgx::ActBuf act(int wtype) const {
        mgx::ActBuf a{};
        a.kind = act_kind(wtype);
        a.stride = max_in;
        a.q = aq; a.d = ad; a.h = ah; a.f = af;
        return a;
    }
    size_t layer_kv() const { return (size_t)n_seq * m->c.heads * cap * 64; }
};

namespace {

size_t row_bytes(int type, int64_t in) {
    switch (type) {
    case mgx::T_F32: return (size_t)in * 4;
    case mgx::T_F16: return (size_t)in * 2;
    case mgx::T_Q8_0: return (size_t)(in / 32) * 34;
    case mgx::T_Q4_0: return (size_t)(in / 32) * 18;
    }
    return 0;
}

const mgx_tensor* find(const mgx_tensor* t, int n, const std::string& name) {
    for (int i = 0; i < n; ++i)
        if (t[i].name && name == t[i].name) return &t[i];
    return nullptr;
}

const mgx_tensor& need(const mgx_tensor* t, int n, const std::string& name, int64_t ne0, int64_t ne1) {
    const mgx_tensor* x = find(t, n, name);
    if (!x) throw Error(MGX_ERR_INVALID, "missing tensor " + name);
    if (x->ne[0] != ne0 || x->ne[1] != ne1 || (x->ne[2] > 1) || (x->ne[3] > 1))
        throw Error(MGX_ERR_INVALID, "bad shape for " + name);
    if (!x->data) throw Error(MGX_ERR_INVALID, "no data for " + name);
    const size_t rb = row_bytes(x->type, ne0);
    if (!rb) throw Error(MGX_ERR_INVALID, "unsupported tensor type for " + name);
    if ((x->type == mgx::T_Q8_0 || x->type == mgx::T_Q4_0) && ne0 % 32)
        throw Error(MGX_ERR_INVALID, name + ": quantized rows must hold whole 32-blocks");
    if (x->nbytes && x->nbytes < rb * (size_t)ne1) throw Error(MGX_ERR_INVALID, "short data for " + name);
    return *x;
}

// Uploads `rows` rows of one ggml tensor into `dst` starting at row `row0` (dst already sized).
void upload_rows(mgx_model* m, const mgx_tensor& t, mgx::DevMat& dst, int64_t row0, hipStream_t s) {
    const int64_t rows = t.ne[1];
    const int in = (int)t.ne[0];
    const size_t rb = row_bytes(t.type, in);
    if (t.type == mgx::T_F32 || t.type == mgx::T_F16) {
        const size_t es = t.type == mgx::T_F32 ? 4 : 2;
        HIP_OK(hipMemcpyAsync((uint8_t*)dst.q + (size_t)row0 * in * es, t.data, rb * rows, hipMemcpyHostToDevice, s));
        return;
    }
    uint8_t* raw = nullptr;
    HIP_OK(hipMalloc(&raw, rb * rows));
    HIP_OK(hipMemcpyAsync(raw, t.data, rb * rows, hipMemcpyHostToDevice, s));
    const size_t qrow = t.type == mgx::T_Q8_0 ? (size_t)in : (size_t)in / 2;
    mgx::launch_repack(t.type, raw, rows, in, (uint8_t*)dst.q + (size_t)row0 * qrow,
                       (uint16_t*)dst.d + (size_t)row0 * (in / 32), s);
    HIP_OK(hipGetLastError());
    HIP_OK(hipStreamSynchronize(s));
    HIP_OK(hipFree(raw));
}

mgx::DevMat alloc_mat(mgx_model* m, int type, int in, int out) {
    mgx::DevMat d{};
    d.type = type; d.in = in; d.out = out;
    switch (type) {
    case mgx::T_Q8_0: d.q = m->mem.alloc<int8_t>((size_t)in * out); d.d = m->mem.alloc<uint16_t>((size_t)(in / 32) * out); break;
    case mgx::T_Q4_0: d.q = m->mem.alloc<uint8_t>((size_t)in / 2 * out); d.d = m->mem.alloc<uint16_t>((size_t)(in / 32) * out); break;
    case mgx::T_F16: d.q = m->mem.alloc<uint16_t>((size_t)in * out); break;
    default: d.q = m->mem.alloc<float>((size_t)in * out); break;
    }
    return d;
}

mgx::DevMat load_mat(mgx_model* m, const mgx_tensor* t, int n, const std::string& name, int in, int out, hipStream_t s) {
    const mgx_tensor& x = need(t, n, name, in, out);
    mgx::DevMat d = alloc_mat(m, x.type, in, out);
    upload_rows(m, x, d, 0, s);
    return d;
}

const float* load_vec(mgx_model* m, const mgx_tensor* t, int n, const std::string& name, int len, hipStream_t s) {
    const mgx_tensor* x = find(t, n, name);
    if (!x || x->type != mgx::T_F32 || x->ne[0] != len || !x->data)
        throw Error(MGX_ERR_INVALID, "missing or bad f32 vector " + name);
    float* d = m->mem.alloc<float>((size_t)len);
    HIP_OK(hipMemcpyAsync(d, x->data, sizeof(float) * (size_t)len, hipMemcpyHostToDevice, s));
    return d;
}

// sin_positions (lm.h:102-116) for positions 0..n-1, computed on the host exactly as the
// reference does (double pow/cos/sin, rounded to float) and kept resident.
std::vector<float> sin_table(int n, const mgx_lm_config& c) {
    const int half = c.dim / 2;
    const double denom = (double)c.pos_denominator;
    std::vector<float> out((size_t)c.dim * n);
    for (int t = 0; t < n; ++t) {
        float* dst = out.data() + (size_t)t * c.dim;
        const double pos = (double)t;
        for (int i = 0; i < half; ++i) {
            const double phase = pos / std::pow((double)c.max_period, (double)i / denom);
            dst[i] = (float)std::cos(phase);
            dst[half + i] = (float)std::sin(phase);
        }
    }
    return out;
}

// One projection of `ncol` activation columns already in s->act(type).
void gemv(mgx_stream* s, const mgx::DevMat& w, int ncol, const mgx::GemvOut& o) {
    mgx::GemvArgs a{};
    a.w = w; a.act = s->act(w.type); a.ncol = ncol; a.o = o;
    mgx::launch_gemv(a, s->hs);
}

mgx::GemvOut out_store(float* y, int stride) { mgx::GemvOut o{}; o.mode = mgx::EPI_STORE; o.y = y; o.y_stride = stride; return o; }
mgx::GemvOut out_resid(float* y, int stride) { mgx::GemvOut o{}; o.mode = mgx::EPI_RESID; o.y = y; o.y_stride = stride; return o; }
mgx::GemvOut out_gelu(float* y, int stride) { mgx::GemvOut o{}; o.mode = mgx::EPI_GELU; o.y = y; o.y_stride = stride; return o; }

void ln_act(mgx_stream* s, const float* x, int ncol, const float* w, const float* b, int wtype) {
    mgx::LnArgs a{};
    a.x = x; a.x_stride = s->m->c.dim; a.dim = s->m->c.dim; a.w = w; a.b = b; a.eps = s->m->c.norm_eps;
    a.out = s->act(wtype);
    mgx::launch_ln_act(a, ncol, s->hs);
}

void to_act(mgx_stream* s, const float* x, int x_stride, int n, int ncol, int wtype) {
    mgx::ActArgs a{};
    a.x = x; a.x_stride = x_stride; a.n = n; a.out = s->act(wtype);
    mgx::launch_act(a, ncol, s->hs);
}

// One sequence step at cache position `position` for every stream: ids of codebook q at
// ids[q * ids_stride]. With `heads`, ends with the logits of this step in s->logits.
void step(mgx_stream* s, const int32_t* ids, int ids_stride, int position, bool heads) {
    const mgx_model* m = s->m;
    const mgx_lm_config& c = m->c;
    const int N = s->n_seq, D = c.dim;
    mgx::EmbedArgs e{};
    for (int q = 0; q < c.n_q; ++q) e.emb[q] = m->emb[q];
    e.n_q = c.n_q; e.ids = ids; e.ids_stride = ids_stride; e.pos = s->pos; e.position = position;
    e.dim = D; e.x = s->x; e.ncol = N;
    mgx::launch_embed(e, s->hs);
    const float scale = 1.0f / std::sqrt((float)c.head_dim);
    for (int l = 0; l < c.layers; ++l) {
        const LayerW& L = m->L[(size_t)l];
        float* Kl = s->K + (size_t)l * s->layer_kv();
        float* Vl = s->V + (size_t)l * s->layer_kv();
        // self-attention
        ln_act(s, s->x, N, L.n1w, L.n1b, L.w[P_QKV].type);
        mgx::GemvOut oq{};
        oq.mode = mgx::EPI_QKV; oq.y = s->qb; oq.k = Kl; oq.v = Vl; oq.dim = D; oq.heads = c.heads;
        oq.cap = s->cap; oq.position = position;
        gemv(s, L.w[P_QKV], N, oq);
        mgx::AttnArgs at{};
        at.q = s->qb; at.k = Kl; at.v = Vl; at.scores = s->scores; at.opart = s->opart; at.dim = D;
        at.heads = c.heads; at.cap = s->cap; at.position = position; at.max_chunks = s->max_chunks;
        at.ncol = N; at.scale = scale;
        mgx::launch_attention(at, s->act(L.w[P_OUT].type), s->hs);
        gemv(s, L.w[P_OUT], N, out_resid(s->x, D));
        // cross-attention, conditional stream only (the null stream's contribution is 0)
        if (s->cross) {
            ln_act(s, s->x, 1, L.ncw, L.ncb, L.w[P_CQ].type);
            gemv(s, L.w[P_CQ], 1, out_store(s->qc, D));
            mgx::XAttnArgs xa{};
            xa.q = s->qc; xa.k = s->xk + (size_t)l * c.heads * s->n_ctx * 64;
            xa.v = s->xv + (size_t)l * c.heads * s->n_ctx * 64; xa.o = s->oc; xa.n_ctx = s->n_ctx; xa.scale = scale;
            mgx::launch_xattn(xa, c.heads, s->hs);
            to_act(s, s->oc, D, D, 1, L.w[P_COUT].type);
            gemv(s, L.w[P_COUT], 1, out_resid(s->x, D));
        }
        // feed-forward
        ln_act(s, s->x, N, L.n2w, L.n2b, L.w[P_FF0].type);
        gemv(s, L.w[P_FF0], N, out_gelu(s->ff, c.ff_dim));
        to_act(s, s->ff, c.ff_dim, c.ff_dim, N, L.w[P_FF2].type);
        gemv(s, L.w[P_FF2], N, out_resid(s->x, D));
    }
    if (heads) {
        ln_act(s, s->x, N, m->out_w, m->out_b, m->heads.type);
        gemv(s, m->heads, N, out_store(s->logits, c.n_q * c.card));
    }
}

void check_config(const mgx_lm_config& c) {
    if (c.dim != c.heads * c.head_dim) throw Error(MGX_ERR_INVALID, "LM dim does not equal heads * head_dim");
    if (c.special_token_id != c.card) throw Error(MGX_ERR_INVALID, "special_token_id should be card: it is the extra embedding row");
    if (c.head_dim != 64) throw Error(MGX_ERR_INVALID, "the decode kernels need head_dim 64");
    if (c.dim % 64 || c.ff_dim % 64) throw Error(MGX_ERR_INVALID, "dim and ff_dim must be multiples of 64");
    if (c.n_q <= 0 || c.n_q > 8) throw Error(MGX_ERR_INVALID, "n_q must be in [1, 8]");
    if (c.card <= 0 || c.card > mgx::MAX_CARD) throw Error(MGX_ERR_INVALID, "card must be in [1, 2048]");
    if (c.layers <= 0 || c.cond_dim <= 0 || c.cond_dim % 32) throw Error(MGX_ERR_INVALID, "bad layers or cond_dim");
}

void make_stream(mgx_model* m, int capacity, int n_seq, const float* t5, int n_ctx, int cross, mgx_stream** out) {
    const mgx_lm_config& c = m->c;
    if (capacity <= 0 || n_seq <= 0) throw Error(MGX_ERR_INVALID, "the kv cache needs positive dimensions");
    if (n_seq > 16) throw Error(MGX_ERR_INVALID, "at most 16 streams per forward");
    if (cross && (n_ctx <= 0 || !t5)) throw Error(MGX_ERR_INVALID, "the conditioning has no tokens");
    if (cross && n_ctx > 256) throw Error(MGX_ERR_INVALID, "at most 256 conditioning tokens");
    HIP_OK(hipSetDevice(m->device));
    auto s = std::make_unique<mgx_stream>();
    s->m = m; s->cap = capacity; s->n_seq = n_seq; s->cross = cross ? 1 : 0; s->n_ctx = cross ? n_ctx : 0;
    s->max_chunks = (capacity + mgx::ATT_CHUNK - 1) / mgx::ATT_CHUNK;
    s->max_in = std::max(c.dim, std::max(c.ff_dim, c.cond_dim));
    HIP_OK(hipStreamCreateWithFlags(&s->hs, hipStreamNonBlocking));
    const size_t kv = s->layer_kv() * c.layers;
    s->K = s->mem.alloc<float>(kv);
    s->V = s->mem.alloc<float>(kv);
    HIP_OK(hipMemsetAsync(s->K, 0, kv * sizeof(float), s->hs));
    HIP_OK(hipMemsetAsync(s->V, 0, kv * sizeof(float), s->hs));
    s->pos = s->mem.alloc<float>((size_t)capacity * c.dim);
    const std::vector<float> pos = sin_table(capacity, c);
    HIP_OK(hipMemcpyAsync(s->pos, pos.data(), pos.size() * sizeof(float), hipMemcpyHostToDevice, s->hs));
    const int cols = std::max(n_seq, s->n_ctx);
    s->x = s->mem.alloc<float>((size_t)cols * c.dim);
    s->qb = s->mem.alloc<float>((size_t)n_seq * c.dim);
    s->ff = s->mem.alloc<float>((size_t)n_seq * c.ff_dim);
    s->scores = s->mem.alloc<float>((size_t)n_seq * c.heads * capacity);
    s->opart = s->mem.alloc<float>((size_t)n_seq * c.heads * s->max_chunks * 64);
    s->logits = s->mem.alloc<float>((size_t)n_seq * c.n_q * c.card);
    s->qc = s->mem.alloc<float>((size_t)c.dim);
    s->oc = s->mem.alloc<float>((size_t)c.dim);
    s->aq = s->mem.alloc<int8_t>((size_t)cols * s->max_in);
    s->ad = s->mem.alloc<float>((size_t)cols * s->max_in / 32);
    s->ah = s->mem.alloc<uint16_t>((size_t)cols * s->max_in);
    s->af = s->mem.alloc<float>((size_t)cols * s->max_in);
    s->ids = s->mem.alloc<int32_t>((size_t)c.n_q * capacity);
    if (s->cross) {
        // lm.cond_proj . t5 + bias, stream 0 only (pipeline.cpp:144-180), then every layer's
        // cross.kv of it, once.
        const int nc = s->n_ctx;
        float* t5d = s->mem.alloc<float>((size_t)nc * c.cond_dim);
        HIP_OK(hipMemcpyAsync(t5d, t5, sizeof(float) * (size_t)nc * c.cond_dim, hipMemcpyHostToDevice, s->hs));
        float* ctx = s->mem.alloc<float>((size_t)nc * c.dim);
        float* kvp = s->mem.alloc<float>((size_t)nc * 2 * c.dim);
        s->xk = s->mem.alloc<float>((size_t)c.layers * c.heads * nc * 64);
        s->xv = s->mem.alloc<float>((size_t)c.layers * c.heads * nc * 64);
        for (int col = 0; col < nc; ++col) {
            to_act(s.get(), t5d + (size_t)col * c.cond_dim, c.cond_dim, c.cond_dim, 1, m->cond_proj.type);
            gemv(s.get(), m->cond_proj, 1, out_store(ctx + (size_t)col * c.dim, c.dim));
        }
        mgx::launch_add_bias(ctx, m->cond_proj_b, c.dim, nc, s->hs);
        for (int l = 0; l < c.layers; ++l) {
            const mgx::DevMat& w = m->L[(size_t)l].w[P_CKV];
            for (int col = 0; col < nc; ++col) {
                to_act(s.get(), ctx + (size_t)col * c.dim, c.dim, c.dim, 1, w.type);
                gemv(s.get(), w, 1, out_store(kvp + (size_t)col * 2 * c.dim, 2 * c.dim));
            }
            mgx::launch_xkv_split(kvp, nc, c.dim, s->xk + (size_t)l * c.heads * nc * 64,
                                  s->xv + (size_t)l * c.heads * nc * 64, s->hs);
        }
    }
    HIP_OK(hipGetLastError());
    HIP_OK(hipStreamSynchronize(s->hs));
    *out = s.release();
}

}  // namespace

extern "C" {

const char* mgx_last_error(void) { return g_error.c_str(); }

int32_t mgx_use_guidance(float cfg_coef, int32_t description_empty) { return cfg_coef != 0.0f && !description_empty; }

int mgx_model_create(const mgx_lm_config* cfg, const mgx_tensor* t, int32_t n, mgx_model** out) {
    return guarded([&] {
        if (!cfg || !t || !out) throw Error(MGX_ERR_INVALID, "null argument");
        *out = nullptr;
        check_config(*cfg);
        auto m = std::make_unique<mgx_model>();
        m->c = *cfg;
        const mgx_lm_config& c = *cfg;
        HIP_OK(hipGetDevice(&m->device));
        hipStream_t s;
        HIP_OK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
        struct StreamGuard { hipStream_t s; ~StreamGuard() { (void)hipStreamSynchronize(s); (void)hipStreamDestroy(s); } } sg{s};
        for (int q = 0; q < c.n_q; ++q)
            m->emb[q] = load_mat(m.get(), t, n, "lm.emb." + std::to_string(q) + ".weight", c.dim, c.card + 1, s);
        // The n_q heads as one [n_q*card][dim] matrix: logits land as [n_q][card] per stream.
        {
            const mgx_tensor& h0 = need(t, n, "lm.head.0.weight", c.dim, c.card);
            m->heads = alloc_mat(m.get(), h0.type, c.dim, c.n_q * c.card);
            for (int q = 0; q < c.n_q; ++q) {
                const mgx_tensor& h = need(t, n, "lm.head." + std::to_string(q) + ".weight", c.dim, c.card);
                if (h.type != h0.type) throw Error(MGX_ERR_INVALID, "the output heads must share one type");
                upload_rows(m.get(), h, m->heads, (int64_t)q * c.card, s);
            }
        }
        m->cond_proj = load_mat(m.get(), t, n, "lm.cond_proj.weight", c.cond_dim, c.dim, s);
        m->cond_proj_b = load_vec(m.get(), t, n, "lm.cond_proj.bias", c.dim, s);
        m->out_w = load_vec(m.get(), t, n, "lm.out_norm.weight", c.dim, s);
        m->out_b = load_vec(m.get(), t, n, "lm.out_norm.bias", c.dim, s);
        m->L.resize((size_t)c.layers);
        for (int i = 0; i < c.layers; ++i) {
            LayerW& L = m->L[(size_t)i];
            const std::string p = "lm." + std::to_string(i) + ".";
            const int ins[P_COUNT] = {c.dim, c.dim, c.dim, c.dim, c.dim, c.dim, c.ff_dim};
            const int outs[P_COUNT] = {3 * c.dim, c.dim, c.dim, 2 * c.dim, c.dim, c.ff_dim, c.dim};
            for (int k = 0; k < P_COUNT; ++k) L.w[k] = load_mat(m.get(), t, n, p + PROJ[k] + ".weight", ins[k], outs[k], s);
            L.n1w = load_vec(m.get(), t, n, p + "norm1.weight", c.dim, s);
            L.n1b = load_vec(m.get(), t, n, p + "norm1.bias", c.dim, s);
            L.ncw = load_vec(m.get(), t, n, p + "norm_cross.weight", c.dim, s);
            L.ncb = load_vec(m.get(), t, n, p + "norm_cross.bias", c.dim, s);
            L.n2w = load_vec(m.get(), t, n, p + "norm2.weight", c.dim, s);
            L.n2b = load_vec(m.get(), t, n, p + "norm2.bias", c.dim, s);
        }
        HIP_OK(hipStreamSynchronize(s));
        *out = m.release();
    });
}

int mgx_model_set_adapters(mgx_model* model, const mgx_adapter* adapters, int32_t n) {
    return guarded([&] {
        if (!model) throw Error(MGX_ERR_INVALID, "null model");
        if (n != 0 || adapters) throw Error(MGX_ERR_INVALID, "adapters are not supported by this build yet");
    });
}

void mgx_model_destroy(mgx_model* model) { delete model; }

int mgx_stream_create(mgx_model* model, int32_t capacity, int32_t n_seq, const float* t5_hidden, int32_t n_ctx,
                      int32_t cross_attention, mgx_stream** out) {
    return guarded([&] {
        if (!model || !out) throw Error(MGX_ERR_INVALID, "null argument");
        *out = nullptr;
        make_stream(model, capacity, n_seq, t5_hidden, n_ctx, cross_attention, out);
    });
}

int mgx_forward(mgx_stream* s, const int32_t* ids, int32_t n_tokens, float* logits_out) {
    return guarded([&] {
        if (!s || !ids) throw Error(MGX_ERR_INVALID, "null argument");
        const mgx_lm_config& c = s->m->c;
        if (n_tokens <= 0) throw Error(MGX_ERR_INVALID, "n_tokens must be positive");
        if (n_tokens > 1 && s->used != 0) throw Error(MGX_ERR_STATE, "multi-token forwards are only supported as a prefill");
        if (s->used + n_tokens > s->cap)
            throw Error(MGX_ERR_OVERFLOW, "kv cache overflow: the sequence is longer than its capacity");
        for (int64_t i = 0; i < (int64_t)c.n_q * n_tokens; ++i)
            if (ids[i] < 0 || ids[i] > c.card) throw Error(MGX_ERR_INVALID, "token id out of range");
        HIP_OK(hipSetDevice(s->m->device));
        HIP_OK(hipMemcpyAsync(s->ids, ids, sizeof(int32_t) * (size_t)c.n_q * n_tokens, hipMemcpyHostToDevice, s->hs));
        // A prefill is the same per-position arithmetic as single steps (its causal mask only
        // adds exact zeros), so the tokens run one position at a time.
        for (int t = 0; t < n_tokens; ++t) step(s, s->ids + t, n_tokens, s->used + t, t == n_tokens - 1);
        HIP_OK(hipGetLastError());
        if (logits_out)
            HIP_OK(hipMemcpyAsync(logits_out, s->logits, sizeof(float) * (size_t)s->n_seq * c.n_q * c.card,
                                  hipMemcpyDeviceToHost, s->hs));
        HIP_OK(hipStreamSynchronize(s->hs));
        s->used += n_tokens;
        s->forwards += 1;
    });
}

int mgx_stream_reset(mgx_stream* s) {
    return guarded([&] {
        if (!s) throw Error(MGX_ERR_INVALID, "null stream");
        s->used = 0;
    });
}
int32_t mgx_stream_used(const mgx_stream* s) { return s ? s->used : -1; }
int32_t mgx_stream_forwards(const mgx_stream* s) { return s ? s->forwards : -1; }
uint64_t mgx_stream_cache_bytes(const mgx_stream* s) {
    return s ? (uint64_t)s->m->c.layers * 2 * 64 * s->cap * s->m->c.heads * s->n_seq * sizeof(float) : 0;
}
void mgx_stream_destroy(mgx_stream* s) { delete s; }

int mgx_generate(mgx_model* m, const float* t5_hidden, int32_t n_ctx, int32_t description_empty,
                 const int32_t* prompt, int32_t prompt_len, const mgx_generate_params* p,
                 int32_t* codes_out, float* first_logits_out, float* step_logits_out, mgx_generate_report* rep) {
    return guarded([&] {
        if (!m || !p || !codes_out || !rep) throw Error(MGX_ERR_INVALID, "null argument");
        const mgx_lm_config& c = m->c;
        const int K = c.n_q, T = p->max_gen_len;
        if (T <= 0) throw Error(MGX_ERR_INVALID, "max_gen_len must be positive");
        if (prompt_len < 0 || prompt_len >= T) throw Error(MGX_ERR_INVALID, "the prompt must be shorter than the generation");
        if (prompt_len > 0 && !prompt) throw Error(MGX_ERR_INVALID, "prompt codes do not hold n_q * prompt_len values");
        if (n_ctx <= 0) throw Error(MGX_ERR_INVALID, "the conditioning has no tokens");
        for (int64_t i = 0; i < (int64_t)K * prompt_len; ++i)
            if (prompt[i] < 0 || prompt[i] >= c.card) throw Error(MGX_ERR_INVALID, "prompt code out of range");
        // DelayPattern with delays 0..n_q-1 (pattern.h:31-115): S = T + n_q, start = P + 1.
        const int S = 1 + T + (K - 1), start = prompt_len + 1;
        auto at = [&](int q, int s) { const int t = s - 1 - q; return (s > 0 && t >= 0 && t < T) ? t : -1; };
        std::vector<int32_t> seq((size_t)K * S, c.special_token_id);
        std::vector<uint8_t> mask((size_t)K * S, 0);
        for (int q = 0; q < K; ++q)
            for (int s = 0; s < S; ++s) {
                const int t = at(q, s);
                if (t < 0) continue;
                mask[(size_t)q * S + s] = 1;
                seq[(size_t)q * S + s] = t < prompt_len ? prompt[(size_t)q * prompt_len + t] : -1;
            }
        const bool guided = mgx_use_guidance(p->cfg_coef, description_empty) != 0;
        const bool sampling = p->use_sampling && p->temperature > 0.0f;
        // The reference draws one uniform per sampled slot, step by step and codebook by
        // codebook; which slots draw depends only on the mask, so the stream is fixed here.
        std::vector<float> uni((size_t)S * K, 0.0f);
        {
            std::mt19937 g((uint32_t)p->seed);
            if (sampling)
                for (int s = start; s < S; ++s)
                    for (int q = 0; q < K; ++q)
                        if (mask[(size_t)q * S + s]) uni[(size_t)s * K + q] = ((g() >> 8) + 0.5f) * (1.0f / 16777216.0f);
        }
        mgx_stream* raw = nullptr;
        make_stream(m, S, guided ? 2 : 1, t5_hidden, n_ctx, guided ? 1 : 0, &raw);
        std::unique_ptr<mgx_stream> s(raw);
        DevArena mem;
        struct Rel { DevArena& a; ~Rel() { a.release(); } } rel{mem};
        int32_t* dseq = mem.alloc<int32_t>(seq.size());
        uint8_t* dmask = mem.alloc<uint8_t>(mask.size());
        float* duni = mem.alloc<float>(uni.size());
        float* dfirst = mem.alloc<float>((size_t)K * c.card);
        float* dsteps = step_logits_out ? mem.alloc<float>((size_t)(S - start) * K * c.card) : nullptr;
        HIP_OK(hipMemcpyAsync(dseq, seq.data(), seq.size() * 4, hipMemcpyHostToDevice, s->hs));
        HIP_OK(hipMemcpyAsync(dmask, mask.data(), mask.size(), hipMemcpyHostToDevice, s->hs));
        HIP_OK(hipMemcpyAsync(duni, uni.data(), uni.size() * 4, hipMemcpyHostToDevice, s->hs));
        HIP_OK(hipStreamSynchronize(s->hs));
        mgx::SampleArgs sa{};
        sa.logits = s->logits; sa.n_q = K; sa.card = c.card; sa.guided = guided; sa.cfg_coef = p->cfg_coef;
        sa.mask = dmask; sa.steps = S; sa.use_sampling = p->use_sampling; sa.temperature = p->temperature;
        sa.top_k = p->top_k; sa.uniforms = duni; sa.special = c.special_token_id; sa.seq = dseq;
        rep->prefill_tokens = start;
        rep->decode_steps = S - start - 1;
        double t0 = now_s();
        for (int offset = start; offset < S; ++offset) {
            if (offset == start)
                for (int pos = 0; pos < start; ++pos) step(s.get(), dseq + pos, S, pos, pos == start - 1);
            else
                step(s.get(), dseq + (offset - 1), S, offset - 1, true);
            sa.offset = offset;
            sa.first_logits = offset == start ? dfirst : nullptr;
            sa.step_logits = dsteps ? dsteps + (size_t)(offset - start) * K * c.card : nullptr;
            mgx::launch_sample(sa, s->hs);
            if (offset == start) {
                HIP_OK(hipGetLastError());
                HIP_OK(hipStreamSynchronize(s->hs));
                rep->prefill_seconds = now_s() - t0;
                t0 = now_s();
            }
        }
        HIP_OK(hipGetLastError());
        HIP_OK(hipStreamSynchronize(s->hs));
        rep->decode_seconds = now_s() - t0;
        s->used = S;
        s->forwards = S - start;
        rep->forwards = S - start;
        rep->cache_bytes = mgx_stream_cache_bytes(s.get());
        HIP_OK(hipMemcpy(seq.data(), dseq, seq.size() * 4, hipMemcpyDeviceToHost));
        if (first_logits_out) HIP_OK(hipMemcpy(first_logits_out, dfirst, sizeof(float) * (size_t)K * c.card, hipMemcpyDeviceToHost));
        if (step_logits_out)
            HIP_OK(hipMemcpy(step_logits_out, dsteps, sizeof(float) * (size_t)(S - start) * K * c.card, hipMemcpyDeviceToHost));
        // revert_pattern_sequence + the final check (pipeline.cpp:307-313)
        for (size_t i = 0; i < (size_t)K * T; ++i) codes_out[i] = c.special_token_id;
        for (int q = 0; q < K; ++q)
            for (int s2 = 0; s2 < S; ++s2) {
                const int t = at(q, s2);
                if (t >= 0) codes_out[(size_t)q * T + t] = seq[(size_t)q * S + s2];
            }
        for (size_t i = 0; i < (size_t)K * T; ++i)
            if (codes_out[i] < 0 || codes_out[i] >= c.card)
                throw Error(MGX_ERR_INVALID, "the generated sequence has a position the pattern never filled");
    });
}

}  // extern "C"
