// runtime.cpp -- the C ABI of include/mgx.h: weights, streams (Decoder), forward and the
// generation loop, all driving the kernels of kernels.hip on one HIP stream.
//
// Reference counterparts: GgufModel / load_gguf (src/gguf_model.h:241-414), LmConfig::from
// (src/mg/lm.h:60-90), Decoder (src/mg/pipeline.cpp:36-195), mg_generate (pipeline.cpp:
// 199-314), KvCache (src/mg/kv_cache.h:33-115), Rng (src/rng.h:15-33), DelayPattern
// (src/mg/pattern.h:31-115).
#include "mgx.h"
#include "kernels.h"
#include "host.h"

#include <hip/hip_runtime.h>

#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <algorithm>
#include <atomic>
#include <map>
#include <memory>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

using namespace mgxh;

namespace {

enum { P_QKV, P_OUT, P_CQ, P_CKV, P_COUT, P_FF0, P_FF2, P_COUNT };
const char* const PROJ[P_COUNT] = {"self.qkv", "self.out", "cross.q", "cross.kv", "cross.out", "ff.0", "ff.2"};

int act_kind(int wtype) {
    return (wtype == mgx::T_Q8_0 || wtype == mgx::T_Q4_0) ? mgx::ACT_Q8 : (wtype == mgx::T_F16 ? mgx::ACT_F16 : mgx::ACT_F32);
}

}  // namespace

// One adapted projection on the device (ac::LoraProjection, lora.h:39-47): A as an f32
// matrix of `rank` rows, B [out][rank], DoRA magnitude and the fixed row norms
// ||W + s*BA|| (lora.h:11-32), s = alpha / rank (times the strength for plain LoRA,
// lora.h:142); DoRA blends with the strength after the row scaling.
struct AdapterW {
    mgx::DevMat A{};
    const float* B = nullptr;
    const float* m = nullptr;
    float* norm = nullptr;
    int rank = 0;
    float scale = 0.0f, strength = 1.0f;
};

struct LayerW {
    mgx::DevMat w[P_COUNT];
    const float *n1w, *n1b, *ncw, *ncb, *n2w, *n2b;
    const AdapterW* ad[P_COUNT] = {};   // null: no adapter, or one that is the identity
};

struct mgx_model {
    mgx_lm_config c{};
    int device = 0;
    DevArena mem;
    mgx::DevMat emb[8]{}, heads{}, cond_proj{};
    const float *cond_proj_b = nullptr, *out_w = nullptr, *out_b = nullptr;
    std::vector<LayerW> L;
    DevArena ad_mem;                 // adapter tensors, replaced as a whole by set_adapters
    std::vector<AdapterW> ads;
    int ad_rank_max = 0;
    std::atomic<int> live{0};        // streams (and sessions) using the model
    ~mgx_model() { ad_mem.release(); mem.release(); }
};

// Device buffers of activation columns in one of the three forms (Q8_0 blocks, fp16, f32).
struct ActStore {
    int8_t* q = nullptr;
    float* d = nullptr;
    uint16_t* h = nullptr;
    float* f = nullptr;
    int stride = 0, cols = 0;   // width, and the columns allocated
    // bm: Q8 block-major, the layout a matrix-core GEMV reads (16 column slots are allocated)
    mgx::ActBuf view(int wtype, bool bm = false) const {
        mgx::ActBuf a{};
        a.kind = act_kind(wtype);
        a.stride = stride;
        a.q = q; a.d = d; a.h = h; a.f = f;
        a.bm = bm && a.kind == mgx::ACT_Q8 ? 1 : 0;
        return a;
    }
};

struct mgx_stream {
    mgx_model* m = nullptr;
    int cap = 0, n_seq = 0, cross = 0, n_ctx = 0, used = 0, forwards = 0, max_chunks = 0;
    int n_req = 1, cpr = 1;                  // requests, and columns (streams) per request
    int cshift = 0;                          // column n belongs to request n >> cshift
    int kv_rows = 0;                         // cache rows per head: cap rounded up to whole 256-key spans
    hipStream_t hs = nullptr;
    DevArena mem;
    float *K = nullptr, *V = nullptr;        // per layer [n_seq][H][kv_rows][64]
    float *xk = nullptr, *xv = nullptr;      // per layer [n_req][H][n_ctx][64], each request's stream 0
    float* ax = nullptr;                     // adapter A x of the running projection [n_seq][rank]
    float* table = nullptr;                  // sinusoid [cap][dim]
    int* dpos = nullptr;                     // [n_req] the position the next step processes
    // Slotted batches: requests join and leave independently. dlive [n_req] (a step advances
    // and samples only live requests), dpar [n_req] their parameters and loop bounds, dnc [n_req]
    // their conditioning lengths (0: no cross-attention). All null for lockstep streams.
    int* dlive = nullptr;
    mgx::ReqParams* dpar = nullptr;
    int* dnc = nullptr;
    float *t5d = nullptr, *ctx = nullptr, *kvp = nullptr;   // memory projection scratch (n_ctx rows)
    float* cmax = nullptr;                   // [n_seq][H][max_chunks] attention chunk maxima
    double* csum = nullptr;                  // [n_seq][H][max_chunks] attention chunk sums
    float *x = nullptr, *qb = nullptr, *opart = nullptr, *logits = nullptr;
    float* qc = nullptr;                     // cross q [n_req][dim]
    ActStore act_o, act_c, act_f;            // attention out, cross-attention out, GELU out
    ActStore act_ln;                         // LayerNorm'd columns in Q8 form (matrix-core GEMVs)
    int32_t* ids = nullptr;                  // [n_q][cap] staged ids for mgx_forward
    // Launch timing: when `prof_on`, every GEMV and attention launch gets a slot in `stamps`
    // (device [slot][2]: earliest block start, latest wave end on the GPU wall clock).
    struct Mark { int slot, kind, tag; double bytes; };
    static constexpr int STAMP_SLOTS = 8192;    // launches; STAMP_SUB sub-slots of 16 B each
    bool prof_on = false;
    int prof_pos = 0;                        // host view of the position, for profiling
    int prof_tag = -1;                       // the projection (MGX_PROF_*) the next launches belong to
    std::vector<Mark> marks;
    unsigned long long* stamps = nullptr;
    double clock_khz = 0.0;
    // A prefill view (make_prefill_view) borrows the caches, the memory, the sinusoid table and
    // the HIP stream of the stream it serves, aimed at one of its requests (aim_view): columns
    // map to that request's caches modulo kv_cols, layers step over the served stream's kv_layer
    // cache columns, and every column reads that request's memory.
    int kv_cols = 0, kv_layer = 0;
    bool shared_mem = false, owns_hs = true;
    int mem_reqs = 0;                        // requests the cross K / V hold (n_req unless a view)
    std::unique_ptr<mgx_stream> pf;          // this stream's prefill view, once a prefill used one
    ~mgx_stream() {
        pf.reset();                          // it runs on this stream's hs
        if (hs) (void)hipStreamSynchronize(hs);
        mem.release();
        if (hs && owns_hs) (void)hipStreamDestroy(hs);
        if (m) m->live.fetch_sub(1);
    }
    // the next timing slot, or null when profiling is off or the slots are used up
    unsigned long long* stamp_slot(int kind, double bytes) {
        if (!prof_on || !stamps || (int)marks.size() >= STAMP_SLOTS) return nullptr;
        marks.push_back({(int)marks.size(), kind, prof_tag, bytes});
        return stamps + 2 * mgx::STAMP_SUB * (size_t)marks.back().slot;
    }
    // one layer's K (or V) cache: every cache column's heads x rows (a prefill view steps over
    // the kv_layer columns of the stream it serves)
    size_t layer_kv() const { return (size_t)(kv_layer ? kv_layer : n_seq) * m->c.heads * kv_rows * 64; }
    void alloc_act(ActStore& a, int cols, int stride) {
        if (n_seq >= 3) cols = (std::max(cols, 16) + 15) / 16 * 16;   // block-major Q8: whole 16-column groups
        a.stride = stride;
        a.cols = cols;
        a.q = mem.alloc<int8_t>((size_t)cols * stride);
        a.d = mem.alloc<float>((size_t)cols * stride / 32);
        a.h = mem.alloc<uint16_t>((size_t)cols * stride);
        a.f = mem.alloc<float>((size_t)cols * stride);
        HIP_OK(hipMemsetAsync(a.q, 0, (size_t)cols * stride, hs));
        HIP_OK(hipMemsetAsync(a.d, 0, (size_t)cols * stride / 32 * sizeof(float), hs));
    }
};

namespace {

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

double bytes_per_weight(int type) {
    switch (type) {
    case mgx::T_Q8_0: return 34.0 / 32.0;
    case mgx::T_Q4_0: return 18.0 / 32.0;
    case mgx::T_F16: return 2.0;
    }
    return 4.0;
}

enum { PROF_GEMV = MGX_PROF_GEMV, PROF_ATTN = MGX_PROF_ATTN };

// One projection. Algorithmic bytes of a launch = the weights at their stored precision.
void gemv(mgx_stream* s, mgx::GemvArgs a) {
    if (a.pro == mgx::PRO_ACT && a.src.bm && !mgx::gemv_mf_ok(a))
        throw Error(MGX_ERR_INVALID, "internal: a block-major source for a projection the matrix cores cannot run");
    if (a.epi == mgx::EPI_QKV && !a.pos)
        throw Error(MGX_ERR_INVALID, "internal: a K/V append without its positions");
    a.stamp = s->stamp_slot(PROF_GEMV, (double)a.w.in * a.w.out * bytes_per_weight(a.w.type));
    mgx::launch_gemv(a, s->hs);
}


// A projection with its adapter, if any: A x first, from the column the projection builds
// (its LayerNorm or f32 source; for an activation-form source, `xf` holds the same column in
// f32), then the GEMV adds s * B(Ax) in its epilogue (lora.h:50-83).
void gemv_ad(mgx_stream* s, mgx::GemvArgs a, const AdapterW* ad, const float* xf = nullptr, int xf_stride = 0) {
    // F16 / F32 weights over more columns than one launch's set: the LayerNorm columns (and the
    // adapter's A x) prepared once in their activation form, then activation-source launches --
    // the per-row-block prologue would recompute every column's LayerNorm once per row block
    if (a.pro == mgx::PRO_LN && (a.w.type == mgx::T_F16 || a.w.type == mgx::T_F32) && a.ncol > 4 &&
        s->act_ln.h && a.ncol <= s->act_ln.cols && a.ncol <= s->n_seq && a.w.in <= s->act_ln.stride) {
        mgx::GemvArgs m = a;
        m.pro = mgx::PRO_ACT;
        m.src = s->act_ln.view(a.w.type);
        m.src.stride = a.w.in;
        mgx::GemvArgs p = ga(ad ? ad->A : mgx::DevMat{}, a.ncol);
        p.w.in = a.w.in;
        p.pro = a.pro; p.x = a.x; p.x_stride = a.x_stride; p.ln_w = a.ln_w; p.ln_b = a.ln_b; p.eps = a.eps;
        p.dst = m.src;
        if (ad) { p.y = s->ax; p.y_stride = ad->rank; }
        mgx::launch_act_prep(p, s->hs);
        if (ad) {
            m.ad_ax = s->ax; m.ad_B = ad->B; m.ad_m = ad->m; m.ad_norm = ad->norm; m.ad_rank = ad->rank;
            m.ad_scale = ad->scale; m.ad_strength = ad->strength;
        }
        gemv(s, m);
        return;
    }
    if (a.pro != mgx::PRO_ACT) {
        // the matrix-core GEMV reads its columns in Q8 form: LayerNorm / quantize them (and
        // take the adapter's A x from the same f32 column) in one preparation launch
        mgx::GemvArgs m = a;
        m.pro = mgx::PRO_ACT;
        m.src = s->act_ln.view(mgx::T_Q8_0, true);
        m.src.stride = a.w.in;
        if (s->act_ln.q && a.w.in <= s->act_ln.stride && mgx::gemv_mf_ok(m)) {
            mgx::GemvArgs p = ga(ad ? ad->A : mgx::DevMat{}, a.ncol);
            p.w.in = a.w.in;
            p.pro = a.pro; p.x = a.x; p.x_stride = a.x_stride; p.ln_w = a.ln_w; p.ln_b = a.ln_b; p.eps = a.eps;
            p.dst = m.src;
            if (ad) { p.y = s->ax; p.y_stride = ad->rank; }
            mgx::launch_act_prep(p, s->hs);
            if (ad) {
                m.ad_ax = s->ax; m.ad_B = ad->B; m.ad_m = ad->m; m.ad_norm = ad->norm; m.ad_rank = ad->rank;
                m.ad_scale = ad->scale; m.ad_strength = ad->strength;
            }
            gemv(s, m);
            return;
        }
    }
    if (ad) {
        mgx::GemvArgs b = ga(ad->A, a.ncol);
        if (a.pro == mgx::PRO_ACT) {
            pro_f32(b, xf, xf_stride);
        } else {
            b.pro = a.pro; b.x = a.x; b.x_stride = a.x_stride; b.ln_w = a.ln_w; b.ln_b = a.ln_b; b.eps = a.eps;
        }
        b.y = s->ax; b.y_stride = ad->rank;
        mgx::launch_adapter_ax(b, s->hs);
        a.ad_ax = s->ax; a.ad_B = ad->B; a.ad_m = ad->m; a.ad_norm = ad->norm; a.ad_rank = ad->rank;
        a.ad_scale = ad->scale; a.ad_strength = ad->strength;
    }
    gemv(s, a);
}

// Whether the projection w over ncol activation-form columns runs on the matrix cores (its
// producer then writes block-major Q8).
bool mf_src(const mgx::DevMat& w, int ncol, int epi) {
    mgx::GemvArgs a = ga(w, ncol);
    a.pro = mgx::PRO_ACT; a.epi = epi;
    a.src.kind = act_kind(w.type); a.src.bm = 1; a.src.stride = w.in;
    return mgx::gemv_mf_ok(a);
}

// One sequence step: column n belongs to request r = n / cpr, which runs at the device
// position dpos[r] and whose codebook q id sits at ids[r * ids_req_stride + q * ids_stride + pos
// - ids_base]. With `heads`, the step's logits land in s->logits. `position` is the host's view
// of the largest position: it sizes the attention grids (the kernels read each column's exact
// key count on the device). Ends by advancing the device positions.
int att_chunks(int position) { return position / mgx::ATT_CHUNK + 1; }

void step(mgx_stream* s, const int32_t* ids, int ids_stride, int ids_base, int ids_req_stride, bool heads,
          const mgx::SampleArgs* sample, int position, int ncol = 0) {
    const mgx_model* m = s->m;
    const mgx_lm_config& c = m->c;
    const int N = ncol > 0 ? ncol : s->n_seq, D = c.dim, R = N / s->cpr;
    mgx::EmbedArgs e{};
    for (int q = 0; q < c.n_q; ++q) e.emb[q] = m->emb[q];
    e.n_q = c.n_q; e.ids = ids; e.ids_stride = ids_stride; e.ids_base = ids_base; e.table = s->table;
    e.ids_req_stride = ids_req_stride; e.cols_per_req = s->cpr;
    e.pos = s->dpos; e.dim = D; e.x = s->x; e.ncol = N;
    mgx::launch_embed(e, s->hs);
    const float scale = 1.0f / std::sqrt((float)c.head_dim);
    for (int l = 0; l < c.layers; ++l) {
        const LayerW& L = m->L[(size_t)l];
        const bool bo = mf_src(L.w[P_OUT], N, mgx::EPI_RESID), bc = mf_src(L.w[P_COUT], R, mgx::EPI_RESID);
        const bool bf = mf_src(L.w[P_FF2], N, mgx::EPI_RESID);
        float* Kl = s->K + (size_t)l * s->layer_kv();
        float* Vl = s->V + (size_t)l * s->layer_kv();
        // self-attention: LN1 + qkv with the K/V append, then per 64-key chunk the scores,
        // softmax terms and V, then the chunks combined
        {
            s->prof_tag = MGX_PROF_QKV;
            mgx::GemvArgs a = ga(L.w[P_QKV], N);
            pro_ln(a, s->x, D, L.n1w, L.n1b, c.norm_eps);
            a.epi = mgx::EPI_QKV; a.y = s->qb; a.k = Kl; a.v = Vl; a.dim = D; a.heads = c.heads; a.cap = s->kv_rows;
            a.pos = s->dpos; a.cshift = s->cshift; a.kv_cols = s->kv_cols;
            gemv_ad(s, a, L.ad[P_QKV]);
        }
        {
            s->prof_tag = MGX_PROF_ATTN;
            mgx::AttnArgs at{};
            at.q = s->qb; at.k = Kl; at.v = Vl; at.opart = s->opart; at.cmax = s->cmax; at.csum = s->csum;
            at.dim = D; at.heads = c.heads; at.cap = s->kv_rows; at.max_chunks = s->max_chunks; at.ncol = N;
            at.scale = scale; at.pos = s->dpos; at.cshift = s->cshift; at.kv_cols = s->kv_cols; at.out = s->act_o.view(L.w[P_OUT].type, bo);
            at.out_f = L.ad[P_OUT] ? s->act_o.f : nullptr;
            // f32 K and V of every key attended, every stream
            at.stamp = s->stamp_slot(PROF_ATTN, 2.0 * N * c.heads * (position + 1) * 64 * 4);
            mgx::launch_attention(at, att_chunks(position), s->hs);
        }
        {
            s->prof_tag = MGX_PROF_OUT;
            mgx::GemvArgs a = ga(L.w[P_OUT], N);
            pro_act(a, s->act_o.view(L.w[P_OUT].type, bo));
            epi_store(a, s->x, D, true);
            gemv_ad(s, a, L.ad[P_OUT], s->act_o.f, D);
        }
        // cross-attention, each request's conditional stream only (the null stream's
        // contribution is exactly 0): column r * cpr of x
        if (s->cross) {
            const size_t xl = (size_t)l * s->mem_reqs * c.heads * s->n_ctx * 64;
            s->prof_tag = MGX_PROF_CROSS_Q;
            mgx::GemvArgs a = ga(L.w[P_CQ], R);
            pro_ln(a, s->x, s->cpr * D, L.ncw, L.ncb, c.norm_eps);
            epi_store(a, s->qc, D);
            gemv_ad(s, a, L.ad[P_CQ]);
            mgx::XAttnArgs xa{};
            xa.q = s->qc; xa.k = s->xk + xl; xa.v = s->xv + xl; xa.n_ctx = s->n_ctx; xa.dim = D; xa.scale = scale;
            xa.nc = s->dnc;
            xa.shared_kv = s->shared_mem ? 1 : 0;
            xa.out = s->act_c.view(L.w[P_COUT].type, bc);
            xa.out_f = L.ad[P_COUT] ? s->act_c.f : nullptr;
            s->prof_tag = MGX_PROF_XATTN;
            // f32 K and V of each request's memory rows
            xa.stamp = s->stamp_slot(MGX_PROF_XATTN, 2.0 * R * c.heads * s->n_ctx * 64 * 4);
            mgx::launch_xattn(xa, c.heads, R, s->hs);
            s->prof_tag = MGX_PROF_CROSS_OUT;
            mgx::GemvArgs b = ga(L.w[P_COUT], R);
            pro_act(b, s->act_c.view(L.w[P_COUT].type, bc));
            epi_store(b, s->x, s->cpr * D, true);
            b.gate = s->dnc;   // a slotted request without conditioning keeps its residual as is
            gemv_ad(s, b, L.ad[P_COUT], s->act_c.f, D);
        }
        // feed-forward: LN2 + ff.0 + GELU (quantized in the epilogue), ff.2 + residual
        {
            s->prof_tag = MGX_PROF_FF0;
            mgx::GemvArgs a = ga(L.w[P_FF0], N);
            pro_ln(a, s->x, D, L.n2w, L.n2b, c.norm_eps);
            a.epi = mgx::EPI_GELU_ACT; a.dst = s->act_f.view(L.w[P_FF2].type, bf);
            a.dst_f = L.ad[P_FF2] ? s->act_f.f : nullptr;
            gemv_ad(s, a, L.ad[P_FF0]);
            s->prof_tag = MGX_PROF_FF2;
            mgx::GemvArgs b = ga(L.w[P_FF2], N);
            pro_act(b, s->act_f.view(L.w[P_FF2].type, bf));
            epi_store(b, s->x, D, true);
            gemv_ad(s, b, L.ad[P_FF2], s->act_f.f, c.ff_dim);
        }
    }
    if (heads) {
        s->prof_tag = MGX_PROF_HEADS;
        mgx::GemvArgs a = ga(m->heads, N);
        pro_ln(a, s->x, D, m->out_w, m->out_b, c.norm_eps);
        epi_store(a, s->logits, c.n_q * c.card);
        gemv_ad(s, a, nullptr);
    }
    s->prof_tag = -1;
    if (sample) mgx::launch_sample(*sample, s->hs);
    mgx::launch_advance(s->dpos, s->dlive, s->dpar, R, s->hs);
}

void check_config(const mgx_lm_config& c) {
    if (c.dim != c.heads * c.head_dim) throw Error(MGX_ERR_INVALID, "LM dim does not equal heads * head_dim");
    if (c.special_token_id != c.card) throw Error(MGX_ERR_INVALID, "special_token_id should be card: it is the extra embedding row");
    if (c.head_dim != 64) throw Error(MGX_ERR_INVALID, "the decode kernels need head_dim 64");
    if (c.dim % 64 || c.ff_dim % 64) throw Error(MGX_ERR_INVALID, "dim and ff_dim must be multiples of 64");
    if (c.n_q <= 0 || c.n_q > 8) throw Error(MGX_ERR_INVALID, "n_q must be in [1, 8]");
    if (c.card <= 0 || c.card > mgx::MAX_CARD) throw Error(MGX_ERR_INVALID, "card must be in [1, 2048]");
    if (c.layers <= 0 || c.cond_dim <= 0 || c.cond_dim % 32) throw Error(MGX_ERR_INVALID, "bad layers or cond_dim");
    // LayerNorm / conversion prologues give each lane one 32-element block of a column
    if (c.dim > 2048 || c.cond_dim > 2048) throw Error(MGX_ERR_INVALID, "dim and cond_dim must be at most 2048");
}

// Every tensor the LM reads, checked before any device work (names, shapes, types, sizes).
void validate_tensors(const mgx_lm_config& c, const mgx_tensor* t, int n) {
    const mgx_tensor* h0 = nullptr;
    for (int q = 0; q < c.n_q; ++q) {
        need(t, n, "lm.emb." + std::to_string(q) + ".weight", c.dim, c.card + 1);
        const mgx_tensor& h = need(t, n, "lm.head." + std::to_string(q) + ".weight", c.dim, c.card);
        if (h0 && h.type != h0->type) throw Error(MGX_ERR_INVALID, "the output heads must share one type");
        h0 = &h;
    }
    need(t, n, "lm.cond_proj.weight", c.cond_dim, c.dim);
    auto vec = [&](const std::string& name) {
        const mgx_tensor* x = find(t, n, name);
        if (!x || x->type != mgx::T_F32 || x->ne[0] != c.dim || !x->data)
            throw Error(MGX_ERR_INVALID, "missing or bad f32 vector " + name);
    };
    vec("lm.cond_proj.bias");
    vec("lm.out_norm.weight");
    vec("lm.out_norm.bias");
    for (int i = 0; i < c.layers; ++i) {
        const std::string p = "lm." + std::to_string(i) + ".";
        const int ins[P_COUNT] = {c.dim, c.dim, c.dim, c.dim, c.dim, c.dim, c.ff_dim};
        const int outs[P_COUNT] = {3 * c.dim, c.dim, c.dim, 2 * c.dim, c.dim, c.ff_dim, c.dim};
        for (int k = 0; k < P_COUNT; ++k) need(t, n, p + PROJ[k] + ".weight", ins[k], outs[k]);
        for (const char* nm : {"norm1", "norm_cross", "norm2"}) {
            vec(p + nm + ".weight");
            vec(p + nm + ".bias");
        }
    }
}

// A stream of n_seq columns for n_req requests (n_seq / n_req columns each; column r * cpr is
// request r's conditional stream). With `cross`, t5[r] [n_ctx][cond_dim] is request r's
// conditioning: projected through lm.cond_proj once and through every layer's cross.kv once.
// lm.cond_proj . t5 + bias, stream 0 only (pipeline.cpp:144-180), then every layer's cross.kv
// of it, for request r: its n_ctx rows of the cross K / V (n_ctx <= the stream's rows per head).
void project_memory(mgx_stream* s, int r, const float* t5, int nc) {
    const mgx_model* m = s->m;
    const mgx_lm_config& c = m->c;
    const int R = s->n_req, rows = s->n_ctx;
    HIP_OK(hipMemcpyAsync(s->t5d, t5, sizeof(float) * (size_t)nc * c.cond_dim, hipMemcpyHostToDevice, s->hs));
    // the memory tokens several to a launch (each column summed as alone): all of them over
    // F16 / F32 weights (one launch, the column sets on blockIdx.y), pairs over quantized ones
    // (the vector GEMV: wider sets would go to the matrix cores, whose staging buffers hold only
    // the stream's own columns); one at a time under an adapter (its A x buffer likewise)
    const auto per = [](const mgx::DevMat& w, const AdapterW* ad) {
        return ad ? 1 : (w.type == mgx::T_F16 || w.type == mgx::T_F32) ? 1 << 30 : 2;
    };
    for (int col = 0, k = per(m->cond_proj, nullptr); col < nc; col += k) {
        mgx::GemvArgs a = ga(m->cond_proj, nc - col < k ? nc - col : k);
        pro_f32(a, s->t5d + (size_t)col * c.cond_dim, c.cond_dim);
        epi_store(a, s->ctx + (size_t)col * c.dim, c.dim);
        gemv(s, a);
    }
    mgx::launch_add_bias(s->ctx, m->cond_proj_b, c.dim, nc, s->hs);
    for (int l = 0; l < c.layers; ++l) {
        const AdapterW* ad = m->L[(size_t)l].ad[P_CKV];
        for (int col = 0, k = per(m->L[(size_t)l].w[P_CKV], ad); col < nc; col += k) {
            mgx::GemvArgs a = ga(m->L[(size_t)l].w[P_CKV], nc - col < k ? nc - col : k);
            pro_f32(a, s->ctx + (size_t)col * c.dim, c.dim);
            epi_store(a, s->kvp + (size_t)col * 2 * c.dim, 2 * c.dim);
            gemv_ad(s, a, ad);
        }
        const size_t off = ((size_t)l * R + r) * c.heads * rows * 64;
        mgx::launch_xkv_split(s->kvp, nc, rows, c.dim, s->xk + off, s->xv + off, s->hs);
    }
}

// t5: one conditioning per request, or null to project them later (project_memory).
void make_stream(mgx_model* m, int capacity, int n_seq, int n_req, const float* const* t5, int n_ctx, int cross,
                 mgx_stream** out) {
    const mgx_lm_config& c = m->c;
    if (capacity <= 0 || n_seq <= 0) throw Error(MGX_ERR_INVALID, "the kv cache needs positive dimensions");
    if (n_seq > 16) throw Error(MGX_ERR_INVALID, "at most 16 streams per forward");
    if (n_req <= 0 || n_req > mgx::MAX_REQ || n_seq % n_req) throw Error(MGX_ERR_INVALID, "bad request count");
    if (cross && n_ctx <= 0) throw Error(MGX_ERR_INVALID, "the conditioning has no tokens");
    if (cross && t5)
        for (int r = 0; r < n_req; ++r)
            if (!t5[r]) throw Error(MGX_ERR_INVALID, "the conditioning has no tokens");
    if (cross && n_ctx > 256) throw Error(MGX_ERR_INVALID, "at most 256 conditioning tokens");
    HIP_OK(hipSetDevice(m->device));
    auto s = std::make_unique<mgx_stream>();
    s->m = m;
    m->live.fetch_add(1);
    s->cap = capacity; s->n_seq = n_seq; s->cross = cross ? 1 : 0; s->n_ctx = cross ? n_ctx : 0;
    s->n_req = n_req; s->cpr = n_seq / n_req; s->mem_reqs = n_req;
    // one request: every column (at most 16) maps to 0; batches have 1 or 2 columns a request
    if (n_req > 1 && s->cpr > 2) throw Error(MGX_ERR_INVALID, "at most 2 streams per request");
    s->cshift = n_req == 1 ? 4 : s->cpr - 1;
    const int spans = (capacity + mgx::ATT_SPAN - 1) / mgx::ATT_SPAN;
    if (spans > mgx::ATT_MAX_SPANS) throw Error(MGX_ERR_INVALID, "capacity above 4096 positions");
    s->kv_rows = spans * mgx::ATT_SPAN;
    s->max_chunks = s->kv_rows / mgx::ATT_CHUNK;
    HIP_OK(hipStreamCreateWithFlags(&s->hs, hipStreamNonBlocking));
    const size_t kv = s->layer_kv() * c.layers;
    s->K = s->mem.alloc<float>(kv);
    s->V = s->mem.alloc<float>(kv);
    HIP_OK(hipMemsetAsync(s->K, 0, kv * sizeof(float), s->hs));
    HIP_OK(hipMemsetAsync(s->V, 0, kv * sizeof(float), s->hs));
    s->table = s->mem.alloc<float>((size_t)capacity * c.dim);
    const std::vector<float> tab = sin_table(capacity, c);
    HIP_OK(hipMemcpyAsync(s->table, tab.data(), tab.size() * sizeof(float), hipMemcpyHostToDevice, s->hs));
    s->dpos = s->mem.alloc<int>((size_t)n_req);
    HIP_OK(hipMemsetAsync(s->dpos, 0, sizeof(int) * (size_t)n_req, s->hs));
    s->cmax = s->mem.alloc<float>((size_t)n_seq * c.heads * s->max_chunks);
    s->csum = s->mem.alloc<double>((size_t)n_seq * c.heads * s->max_chunks);
    s->x = s->mem.alloc<float>((size_t)n_seq * c.dim);
    s->qb = s->mem.alloc<float>((size_t)n_seq * c.dim);
    s->opart = s->mem.alloc<float>((size_t)n_seq * c.heads * s->max_chunks * 64);
    s->logits = s->mem.alloc<float>((size_t)n_seq * c.n_q * c.card);
    s->qc = s->mem.alloc<float>((size_t)n_req * c.dim);
    s->alloc_act(s->act_o, n_seq, c.dim);
    s->alloc_act(s->act_c, n_req, c.dim);
    s->alloc_act(s->act_f, n_seq, c.ff_dim);
    if (n_seq >= 3) s->alloc_act(s->act_ln, n_seq, c.dim);
    s->ids = s->mem.alloc<int32_t>((size_t)c.n_q * capacity);
    if (m->ad_rank_max > 0) s->ax = s->mem.alloc<float>((size_t)std::max(n_seq, 2) * m->ad_rank_max);
    if (s->cross) {
        const int nc = s->n_ctx;
        s->t5d = s->mem.alloc<float>((size_t)nc * c.cond_dim);
        s->ctx = s->mem.alloc<float>((size_t)nc * c.dim);
        s->kvp = s->mem.alloc<float>((size_t)nc * 2 * c.dim);
        s->xk = s->mem.alloc<float>((size_t)c.layers * n_req * c.heads * nc * 64);
        s->xv = s->mem.alloc<float>((size_t)c.layers * n_req * c.heads * nc * 64);
        if (t5)
            for (int r = 0; r < n_req; ++r) project_memory(s.get(), r, t5[r], nc);
    }
    HIP_OK(hipGetLastError());
    HIP_OK(hipStreamSynchronize(s->hs));
    *out = s.release();
}

}  // namespace

namespace {

// A view of single-request stream `main` that runs `g` prompt positions at once: g * cpr columns,
// column r * cpr + s is stream s at position dpos[r], appending to and attending main's caches
// (kv_cols = cpr) and reading main's memory. Only the per-column working buffers are its own.
std::unique_ptr<mgx_stream> make_prefill_view(mgx_stream* main, int g) {
    const mgx_model* m = main->m;
    const mgx_lm_config& c = m->c;
    const int cpr = main->cpr, n_seq = g * cpr;
    if (g < 2 || n_seq > mgx::MF_MAX_COLS || (cpr & (cpr - 1))) throw Error(MGX_ERR_INVALID, "internal: bad prefill view shape");
    auto s = std::make_unique<mgx_stream>();
    s->m = main->m;
    s->m->live.fetch_add(1);
    s->cap = main->cap; s->n_seq = n_seq; s->cross = main->cross; s->n_ctx = main->n_ctx;
    s->n_req = g; s->cpr = cpr; s->mem_reqs = main->mem_reqs;
    s->cshift = 0;
    while ((1 << s->cshift) < cpr) ++s->cshift;   // log2(cpr): 1, 2, 4 or 8 streams
    s->max_chunks = main->max_chunks; s->kv_rows = main->kv_rows;
    s->hs = main->hs; s->owns_hs = false;
    s->K = main->K; s->V = main->V; s->xk = main->xk; s->xv = main->xv; s->table = main->table;
    s->kv_cols = cpr; s->kv_layer = main->n_seq; s->shared_mem = true;
    s->dpos = s->mem.alloc<int>((size_t)g);
    if (main->dnc) s->dnc = s->mem.alloc<int>((size_t)g);   // the aimed request's conditioning length, per position
    s->cmax = s->mem.alloc<float>((size_t)n_seq * c.heads * s->max_chunks);
    s->csum = s->mem.alloc<double>((size_t)n_seq * c.heads * s->max_chunks);
    s->x = s->mem.alloc<float>((size_t)n_seq * c.dim);
    s->qb = s->mem.alloc<float>((size_t)n_seq * c.dim);
    s->opart = s->mem.alloc<float>((size_t)n_seq * c.heads * s->max_chunks * 64);
    s->qc = s->mem.alloc<float>((size_t)g * c.dim);
    s->alloc_act(s->act_o, n_seq, c.dim);
    s->alloc_act(s->act_c, g, c.dim);
    s->alloc_act(s->act_f, n_seq, c.ff_dim);
    s->alloc_act(s->act_ln, n_seq, c.dim);
    if (m->ad_rank_max > 0) s->ax = s->mem.alloc<float>((size_t)n_seq * m->ad_rank_max);
    return s;
}

// Aims view pf of stream main at main's request r: its caches (columns r * cpr ..), its memory.
void aim_view(mgx_stream* pf, const mgx_stream* main, int r) {
    const mgx_lm_config& c = main->m->c;
    const size_t col = (size_t)r * main->cpr * c.heads * main->kv_rows * 64;
    pf->K = main->K + col;
    pf->V = main->V + col;
    const size_t mem = (size_t)r * c.heads * main->n_ctx * 64;
    pf->xk = main->xk ? main->xk + mem : nullptr;
    pf->xv = main->xv ? main->xv + mem : nullptr;
}

// Positions per prefill group: MF_MAX_COLS columns (the matrix-core GEMV's widest launch; 512
// columns: c4's prefill 239 ms with 64, 191 with 128, 156 with 256, 145 with 512, 143 with 1024
// and twice the view's scratch).
int prefill_positions(const mgx_stream* s) {
    return mgx::MF_MAX_COLS / s->cpr;
}

// Whether stream s prefills through a view: a view's column n is at position n >> log2(streams)
// (1, 2, 4 or 8 streams per request), and a lockstep batch takes one request at a time only
// when a view's group is wider than the batch's own steps.
bool prefill_by_view(const mgx_stream* s) {
    if (s->cpr > 8 || (s->cpr & (s->cpr - 1))) return false;
    return s->n_req == 1 || prefill_positions(s) * s->cpr > s->n_seq;
}

// Runs positions first .. first + count - 1 of stream s without heads (the positions of a
// prefill before its last), request by request, prefill_positions at a time through s's
// prefill view aimed at the request: each column at its own position, causal by key count, all
// of a group's K / V appended by the same launch before any column attends. Request r's id of
// codebook q at position p is ids[r * ids_req_stride + q * ids_stride + p - ids_base]. Leaves
// every request's device position at first + count. Returns false, running nothing, when the
// stream does not prefill by view (prefill_by_view) or count < 2.
bool run_prefill(mgx_stream* s, const int32_t* ids, int ids_stride, int ids_base, int ids_req_stride, int first,
                 int count) {
    if (!prefill_by_view(s) || count < 2) return false;
    if (!s->pf) s->pf = make_prefill_view(s, prefill_positions(s));
    mgx_stream* pf = s->pf.get();
    const int G = pf->n_req;
    for (int r = 0; r < s->n_req; ++r) {
        aim_view(pf, s, r);
        const int32_t* idr = ids + (size_t)r * ids_req_stride;
        for (int p0 = 0; p0 < count; p0 += G) {
            const int g = std::min(G, count - p0);
            mgx::launch_set_positions(pf->dpos, g, first + p0, s->hs);
            step(pf, idr, ids_stride, ids_base, 0, false, nullptr, first + p0 + g - 1, g * pf->cpr);
        }
    }
    mgx::launch_fill_i32(s->dpos, s->n_req, first + count, s->hs);
    return true;
}

}  // namespace

// library-internal (gguf.cpp): the status/message convention, and a projection's (in, out)
__attribute__((visibility("hidden"))) int mgx_internal_set_error(int code, const char* msg) {
    g_error = msg ? msg : "";
    return code;
}
__attribute__((visibility("hidden"))) bool mgx_internal_proj_shape(const mgx_model* m, const char* name, int64_t* in,
                                                                    int64_t* out) {
    if (!m || !name) return false;
    for (int l = 0; l < m->c.layers; ++l)
        for (int k = 0; k < P_COUNT; ++k)
            if (std::string(name) == "lm." + std::to_string(l) + "." + PROJ[k] + ".weight") {
                *in = m->L[(size_t)l].w[k].in;
                *out = m->L[(size_t)l].w[k].out;
                return true;
            }
    return false;
}

extern "C" {

const char* mgx_last_error(void) { return g_error.c_str(); }

int32_t mgx_use_guidance(float cfg_coef, int32_t description_empty) { return cfg_coef != 0.0f && !description_empty; }

int mgx_model_create(const mgx_lm_config* cfg, const mgx_tensor* t, int32_t n, mgx_model** out) {
    return guarded([&] {
        if (!cfg || !t || !out) throw Error(MGX_ERR_INVALID, "null argument");
        *out = nullptr;
        check_config(*cfg);
        validate_tensors(*cfg, t, n);
        auto m = std::make_unique<mgx_model>();
        m->c = *cfg;
        const mgx_lm_config& c = *cfg;
        HIP_OK(hipGetDevice(&m->device));
        hipStream_t s;
        HIP_OK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
        struct StreamGuard { hipStream_t s; ~StreamGuard() { (void)hipStreamSynchronize(s); (void)hipStreamDestroy(s); } } sg{s};
        for (int q = 0; q < c.n_q; ++q)
            m->emb[q] = load_mat(m->mem, t, n, "lm.emb." + std::to_string(q) + ".weight", c.dim, c.card + 1, s);
        // The n_q heads as one [n_q*card][dim] matrix: logits land as [n_q][card] per stream.
        {
            const mgx_tensor& h0 = need(t, n, "lm.head.0.weight", c.dim, c.card);
            m->heads = alloc_mat(m->mem, h0.type, c.dim, c.n_q * c.card);
            for (int q = 0; q < c.n_q; ++q) {
                const mgx_tensor& h = need(t, n, "lm.head." + std::to_string(q) + ".weight", c.dim, c.card);
                if (h.type != h0.type) throw Error(MGX_ERR_INVALID, "the output heads must share one type");
                upload_rows(h, m->heads, (int64_t)q * c.card, s);
            }
        }
        m->cond_proj = load_mat(m->mem, t, n, "lm.cond_proj.weight", c.cond_dim, c.dim, s);
        m->cond_proj_b = load_vec(m->mem, t, n, "lm.cond_proj.bias", c.dim, s);
        m->out_w = load_vec(m->mem, t, n, "lm.out_norm.weight", c.dim, s);
        m->out_b = load_vec(m->mem, t, n, "lm.out_norm.bias", c.dim, s);
        m->L.resize((size_t)c.layers);
        for (int i = 0; i < c.layers; ++i) {
            LayerW& L = m->L[(size_t)i];
            const std::string p = "lm." + std::to_string(i) + ".";
            const int ins[P_COUNT] = {c.dim, c.dim, c.dim, c.dim, c.dim, c.dim, c.ff_dim};
            const int outs[P_COUNT] = {3 * c.dim, c.dim, c.dim, 2 * c.dim, c.dim, c.ff_dim, c.dim};
            for (int k = 0; k < P_COUNT; ++k) L.w[k] = load_mat(m->mem, t, n, p + PROJ[k] + ".weight", ins[k], outs[k], s);
            L.n1w = load_vec(m->mem, t, n, p + "norm1.weight", c.dim, s);
            L.n1b = load_vec(m->mem, t, n, p + "norm1.bias", c.dim, s);
            L.ncw = load_vec(m->mem, t, n, p + "norm_cross.weight", c.dim, s);
            L.ncb = load_vec(m->mem, t, n, p + "norm_cross.bias", c.dim, s);
            L.n2w = load_vec(m->mem, t, n, p + "norm2.weight", c.dim, s);
            L.n2b = load_vec(m->mem, t, n, p + "norm2.bias", c.dim, s);
        }
        // every Q8_0 projection's matrix-core copies: tile-transposed scales, operand-order quants
        auto with_dt = [&](mgx::DevMat& w) {
            if ((w.type != mgx::T_Q8_0 && w.type != mgx::T_Q4_0) || w.out % 16 || w.in % 32) return;
            uint16_t* dt = m->mem.alloc<uint16_t>((size_t)w.out * (w.in / 32));
            mgx::launch_scales_t(w, dt, s);
            if (w.type == mgx::T_Q8_0) {
                int8_t* qm = m->mem.alloc<int8_t>((size_t)w.out * w.in);
                mgx::launch_weights_mf(w, qm, s);
                w.qm = qm;
            } else {
                uint32_t* qm = m->mem.alloc<uint32_t>((size_t)w.out * w.in / 8);
                mgx::launch_weights_mf4(w, qm, s);
                w.qm = (int8_t*)qm;
            }
            HIP_OK(hipGetLastError());
            w.dt = dt;
        };
        with_dt(m->heads);
        for (LayerW& L : m->L)
            for (int k = 0; k < P_COUNT; ++k) with_dt(L.w[k]);
        HIP_OK(hipStreamSynchronize(s));
        *out = m.release();
    });
}

int mgx_model_set_adapters(mgx_model* model, const mgx_adapter* adapters, int32_t n) {
    return guarded([&] {
        if (!model) throw Error(MGX_ERR_INVALID, "null model");
        if (n < 0 || (n > 0 && !adapters)) throw Error(MGX_ERR_INVALID, "bad adapter list");
        if (model->live.load() != 0)
            throw Error(MGX_ERR_STATE, "adapters can change only while no stream or session uses the model");
        const mgx_lm_config& c = model->c;
        // load_lora / load_mg_lora's checks (lora.h:113-176, 195-210), all before any change
        struct Slot { int layer, proj; };
        std::vector<Slot> slots((size_t)n);
        for (int i = 0; i < n; ++i) {
            const mgx_adapter& a = adapters[i];
            const std::string target = a.target ? a.target : "";
            int li = -1, pi = -1;
            for (int l = 0; l < c.layers && li < 0; ++l)
                for (int k = 0; k < P_COUNT; ++k)
                    if (target == "lm." + std::to_string(l) + "." + PROJ[k] + ".weight") { li = l; pi = k; break; }
            if (li < 0) throw Error(MGX_ERR_INVALID, "unsupported MusicGen adapter target: " + target);
            for (int j = 0; j < i; ++j)
                if (slots[(size_t)j].layer == li && slots[(size_t)j].proj == pi)
                    throw Error(MGX_ERR_INVALID, "two adapters for " + target);
            slots[(size_t)i] = {li, pi};
            if (a.rank <= 0 || !std::isfinite(a.alpha) || a.alpha <= 0 || !std::isfinite(a.strength))
                throw Error(MGX_ERR_INVALID, "invalid adapter rank, alpha or strength");
            if (a.rank > 64) throw Error(MGX_ERR_INVALID, "adapter ranks above 64 are not supported");
            if (!a.A || !a.B) throw Error(MGX_ERR_INVALID, "adapter shape mismatch: " + target);
            const mgx::DevMat& W = model->L[(size_t)li].w[pi];
            for (size_t k = 0; k < (size_t)a.rank * W.in; ++k)
                if (!std::isfinite(a.A[k])) throw Error(MGX_ERR_INVALID, "nonfinite adapter tensor");
            for (size_t k = 0; k < (size_t)W.out * a.rank; ++k)
                if (!std::isfinite(a.B[k])) throw Error(MGX_ERR_INVALID, "nonfinite adapter tensor");
            if (a.magnitude)
                for (int k = 0; k < W.out; ++k)
                    if (!std::isfinite(a.magnitude[k])) throw Error(MGX_ERR_INVALID, "nonfinite adapter tensor");
        }
        HIP_OK(hipSetDevice(model->device));
        for (LayerW& L : model->L)
            for (int k = 0; k < P_COUNT; ++k) L.ad[k] = nullptr;
        model->ad_mem.release();
        model->ads.assign((size_t)n, AdapterW{});
        model->ad_rank_max = 0;
        if (n == 0) return;
        hipStream_t hs;
        HIP_OK(hipStreamCreateWithFlags(&hs, hipStreamNonBlocking));
        struct StreamGuard { hipStream_t s; ~StreamGuard() { (void)hipStreamSynchronize(s); (void)hipStreamDestroy(s); } } sg{hs};
        int* bad = model->ad_mem.alloc<int>(1);
        HIP_OK(hipMemsetAsync(bad, 0, sizeof(int), hs));
        for (int i = 0; i < n; ++i) {
            const mgx_adapter& a = adapters[i];
            AdapterW& w = model->ads[(size_t)i];
            const mgx::DevMat& W = model->L[(size_t)slots[(size_t)i].layer].w[slots[(size_t)i].proj];
            w.rank = a.rank;
            w.scale = (a.magnitude ? 1.0f : a.strength) * a.alpha / (float)a.rank;   // lora.h:142
            w.strength = a.magnitude ? a.strength : 1.0f;
            // a zero-strength adapter leaves the projection as it is (lora.h:62)
            if ((a.magnitude && w.strength == 0.0f) || (!a.magnitude && w.scale == 0.0f)) continue;
            float* A = model->ad_mem.alloc<float>((size_t)a.rank * W.in);
            float* B = model->ad_mem.alloc<float>((size_t)W.out * a.rank);
            HIP_OK(hipMemcpyAsync(A, a.A, sizeof(float) * (size_t)a.rank * W.in, hipMemcpyHostToDevice, hs));
            HIP_OK(hipMemcpyAsync(B, a.B, sizeof(float) * (size_t)W.out * a.rank, hipMemcpyHostToDevice, hs));
            w.A.type = mgx::T_F32; w.A.in = W.in; w.A.out = a.rank; w.A.q = A; w.A.d = nullptr;
            w.B = B;
            if (a.magnitude) {
                float* mg = model->ad_mem.alloc<float>((size_t)W.out);
                HIP_OK(hipMemcpyAsync(mg, a.magnitude, sizeof(float) * (size_t)W.out, hipMemcpyHostToDevice, hs));
                w.m = mg;
                w.norm = model->ad_mem.alloc<float>((size_t)W.out);
                mgx::launch_dora_norm(W, A, B, a.rank, w.scale, w.norm, bad, hs);
                HIP_OK(hipGetLastError());
            }
            model->L[(size_t)slots[(size_t)i].layer].ad[slots[(size_t)i].proj] = &w;
            model->ad_rank_max = std::max(model->ad_rank_max, a.rank);
        }
        int nonfinite = 0;
        HIP_OK(hipMemcpyAsync(&nonfinite, bad, sizeof(int), hipMemcpyDeviceToHost, hs));
        HIP_OK(hipStreamSynchronize(hs));
        if (nonfinite) {
            for (LayerW& L : model->L)
                for (int k = 0; k < P_COUNT; ++k) L.ad[k] = nullptr;
            model->ads.clear();
            model->ad_rank_max = 0;
            model->ad_mem.release();
            throw Error(MGX_ERR_INVALID, "nonfinite DoRA base weight");
        }
    });
}

void mgx_model_destroy(mgx_model* model) { delete model; }

int mgx_stream_create(mgx_model* model, int32_t capacity, int32_t n_seq, const float* t5_hidden, int32_t n_ctx,
                      int32_t cross_attention, mgx_stream** out) {
    return guarded([&] {
        if (!model || !out) throw Error(MGX_ERR_INVALID, "null argument");
        *out = nullptr;
        make_stream(model, capacity, n_seq, 1, &t5_hidden, n_ctx, cross_attention, out);
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
        const int used = s->used;
        HIP_OK(hipMemcpyAsync(s->dpos, &used, sizeof(int), hipMemcpyHostToDevice, s->hs));
        // A prefill is the same per-position arithmetic as single steps (its causal mask only
        // adds exact zeros): the positions before the last run in groups of columns, the last
        // (the only one whose logits are read) as a single step.
        if (run_prefill(s, s->ids, n_tokens, used, 0, used, n_tokens - 1))
            step(s, s->ids, n_tokens, used, 0, true, nullptr, used + n_tokens - 1);
        else
            for (int t = 0; t < n_tokens; ++t) step(s, s->ids, n_tokens, used, 0, t == n_tokens - 1, nullptr, used + t);
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

}  // extern "C"

// ------------------------------------------------------------------------------------
// generation sessions: mg_generate (pipeline.cpp:199-314) cut into resumable pieces
// ------------------------------------------------------------------------------------
// R requests in lockstep (one for mgx_session_create): the same prompt length, generation
// length, conditioning length and guidance; each its own conditioning, prompt, seed and
// sampling parameters, KV cache columns and sampler rows.
struct mgx_session {
    mgx_model* m = nullptr;
    std::unique_ptr<mgx_stream> s;
    DevArena mem;
    int R = 1, K = 0, T = 0, S = 0, start = 0, next = 0;   // next: the next loop offset to run
    bool guided = false;
    std::vector<int32_t> seq;                     // [R][K][S]
    int32_t* dseq = nullptr;
    float *dfirst = nullptr, *dsteps = nullptr;   // [R][K][card], [R][S - start][K][card]
    mgx::SampleArgs sa{};
    double prefill_seconds = 0.0, decode_seconds = 0.0;
    int prof_every = 0;
    // Captured prefill positions (no heads) and decode steps (heads, CFG mix, sampling,
    // position advance), one pair per attention chunk count: every kernel reads the position
    // from the device, so a graph replays for every position with that many 64-key chunks.
    hipGraphExec_t g_body[mgx::ATT_MAX_CHUNKS] = {}, g_step[mgx::ATT_MAX_CHUNKS] = {};
    // MGX_GRAPHS=0 launches the same kernels one by one (for tools that do not follow
    // stream capture, such as kernel tracers).
    bool use_graphs = true;
    ~mgx_session() {
        if (s && s->hs) (void)hipStreamSynchronize(s->hs);
        for (int i = 0; i < mgx::ATT_MAX_CHUNKS; ++i) {
            if (g_body[i]) (void)hipGraphExecDestroy(g_body[i]);
            if (g_step[i]) (void)hipGraphExecDestroy(g_step[i]);
        }
        mem.release();
    }
    int pattern_t(int q, int step) const { const int t = step - 1 - q; return (step > 0 && t >= 0 && t < T) ? t : -1; }
};

namespace {

mgx::ReqParams req_params(const mgx_generate_params& p, bool guided, int start, int steps) {
    mgx::ReqParams r{};
    r.cfg_coef = p.cfg_coef; r.temperature = p.temperature; r.use_sampling = p.use_sampling; r.top_k = p.top_k;
    r.guided = guided ? 1 : 0; r.start = start; r.steps = steps;
    return r;
}

// mg_generate's argument checks (pipeline.cpp:204-212) for one request
void check_request(const mgx_lm_config& c, const mgx_batch_request& q, int n_ctx, int prompt_len) {
    const int T = q.params.max_gen_len;
    if (T <= 0) throw Error(MGX_ERR_INVALID, "max_gen_len must be positive");
    if (prompt_len < 0 || prompt_len >= T) throw Error(MGX_ERR_INVALID, "the prompt must be shorter than the generation");
    if (prompt_len > 0 && !q.prompt_codes) throw Error(MGX_ERR_INVALID, "prompt codes do not hold n_q * prompt_len values");
    if (n_ctx <= 0) throw Error(MGX_ERR_INVALID, "the conditioning has no tokens");
    for (int64_t i = 0; i < (int64_t)c.n_q * prompt_len; ++i)
        if (q.prompt_codes[i] < 0 || q.prompt_codes[i] >= c.card) throw Error(MGX_ERR_INVALID, "prompt code out of range");
}

void session_create(mgx_model* m, const mgx_batch_request* reqs, int R, int32_t n_ctx, int32_t prompt_len,
                    int keep_steps, mgx_session** out) {
    if (!m || !reqs || !out) throw Error(MGX_ERR_INVALID, "null argument");
    *out = nullptr;
    const mgx_lm_config& c = m->c;
    if (R <= 0 || R > mgx::MAX_REQ) throw Error(MGX_ERR_INVALID, "a batch holds 1 to 16 requests");
    const int K = c.n_q, T = reqs[0].params.max_gen_len;
    for (int r = 0; r < R; ++r) {
        const mgx_batch_request& q = reqs[r];
        check_request(c, q, n_ctx, prompt_len);
        if (q.params.max_gen_len != T) throw Error(MGX_ERR_INVALID, "the requests of a batch share max_gen_len");
        if ((mgx_use_guidance(q.params.cfg_coef, q.description_empty) != 0) !=
            (mgx_use_guidance(reqs[0].params.cfg_coef, reqs[0].description_empty) != 0))
            throw Error(MGX_ERR_INVALID, "the requests of a batch are all guided or all unguided");
    }
    auto ss = std::make_unique<mgx_session>();
    ss->m = m; ss->R = R; ss->K = K; ss->T = T;
    if (const char* g = std::getenv("MGX_GRAPHS")) ss->use_graphs = std::strcmp(g, "0") != 0;
    // DelayPattern with delays 0..n_q-1 (pattern.h:31-115): S = T + n_q, start = P + 1.
    ss->S = 1 + T + (K - 1);
    ss->start = prompt_len + 1;
    ss->next = ss->start;
    const int S = ss->S, start = ss->start;
    ss->guided = mgx_use_guidance(reqs[0].params.cfg_coef, reqs[0].description_empty) != 0;
    if (R * (ss->guided ? 2 : 1) > 16) throw Error(MGX_ERR_INVALID, "at most 16 streams per batch (8 guided requests)");
    std::vector<uint8_t> mask((size_t)K * S, 0);
    for (int q = 0; q < K; ++q)
        for (int st = 0; st < S; ++st) mask[(size_t)q * S + st] = ss->pattern_t(q, st) >= 0;
    ss->seq.assign((size_t)R * K * S, c.special_token_id);
    // The reference draws one uniform per sampled slot, step by step and codebook by
    // codebook (pipeline.cpp:278-288, rng.h:20-22); which slots draw depends only on the
    // mask, so each request's whole stream is drawn here.
    std::vector<float> uni((size_t)R * S * K, 0.0f);
    std::vector<mgx::ReqParams> par((size_t)R);
    mgx::SampleArgs& sa = ss->sa;
    for (int r = 0; r < R; ++r) {
        const mgx_batch_request& rq = reqs[r];
        int32_t* seq = ss->seq.data() + (size_t)r * K * S;
        for (int q = 0; q < K; ++q)
            for (int st = 0; st < S; ++st) {
                const int t = ss->pattern_t(q, st);
                if (t >= 0) seq[(size_t)q * S + st] = t < prompt_len ? rq.prompt_codes[(size_t)q * prompt_len + t] : -1;
            }
        const mgx_generate_params& p = rq.params;
        if (p.use_sampling && p.temperature > 0.0f) {
            std::mt19937 g((uint32_t)p.seed);
            float* u = uni.data() + (size_t)r * S * K;
            for (int st = start; st < S; ++st)
                for (int q = 0; q < K; ++q)
                    if (mask[(size_t)q * S + st]) u[(size_t)st * K + q] = ((g() >> 8) + 0.5f) * (1.0f / 16777216.0f);
        }
        par[(size_t)r] = req_params(p, ss->guided, start, S);
    }
    std::vector<const float*> t5s((size_t)R);
    for (int r = 0; r < R; ++r) t5s[(size_t)r] = reqs[r].t5_hidden;
    mgx_stream* raw = nullptr;
    make_stream(m, S, R * (ss->guided ? 2 : 1), R, t5s.data(), n_ctx, ss->guided ? 1 : 0, &raw);
    ss->s.reset(raw);
    mgx_stream* st = ss->s.get();
    if (start - 1 >= 2 && prefill_by_view(st)) st->pf = make_prefill_view(st, prefill_positions(st));
    ss->dseq = ss->mem.alloc<int32_t>(ss->seq.size());
    uint8_t* dmask = ss->mem.alloc<uint8_t>(mask.size());
    mgx::ReqParams* dpar = ss->mem.alloc<mgx::ReqParams>(par.size());
    HIP_OK(hipMemcpyAsync(dpar, par.data(), par.size() * sizeof(mgx::ReqParams), hipMemcpyHostToDevice, st->hs));
    float* duni = ss->mem.alloc<float>(uni.size());
    ss->dfirst = ss->mem.alloc<float>((size_t)R * K * c.card);
    if (keep_steps) ss->dsteps = ss->mem.alloc<float>((size_t)R * (S - start) * K * c.card);
    HIP_OK(hipMemcpyAsync(ss->dseq, ss->seq.data(), ss->seq.size() * 4, hipMemcpyHostToDevice, st->hs));
    HIP_OK(hipMemcpyAsync(dmask, mask.data(), mask.size(), hipMemcpyHostToDevice, st->hs));
    HIP_OK(hipMemcpyAsync(duni, uni.data(), uni.size() * 4, hipMemcpyHostToDevice, st->hs));
    HIP_OK(hipStreamSynchronize(st->hs));
    sa.logits = st->logits; sa.n_q = K; sa.card = c.card; sa.n_req = R; sa.cpr = st->cpr; sa.par = dpar;
    sa.pos = st->dpos; sa.live = nullptr; sa.seq_len = S; sa.mask = dmask; sa.mask_stride = 0;
    sa.special = c.special_token_id; sa.uniforms = duni; sa.seq = ss->dseq;
    sa.first_logits = ss->dfirst; sa.step_logits = ss->dsteps; sa.step_rows = S - start;
    *out = ss.release();
}

hipGraphExec_t capture(mgx_session* ss, bool full, int position) {
    mgx_stream* s = ss->s.get();
    hipGraph_t g = nullptr;
    hipGraphExec_t e = nullptr;
    HIP_OK(hipStreamBeginCapture(s->hs, hipStreamCaptureModeThreadLocal));
    step(s, ss->dseq, ss->S, 0, ss->K * ss->S, full, full ? &ss->sa : nullptr, position);
    HIP_OK(hipStreamEndCapture(s->hs, &g));
    const hipError_t rc = hipGraphInstantiate(&e, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    HIP_OK(rc);
    return e;
}

// One loop iteration's position: the body at a prefill position, or the full step.
void run_position(mgx_session* ss, bool full, bool profiled, int position) {
    mgx_stream* s = ss->s.get();
    if (profiled) {
        s->prof_on = true;
        s->prof_pos = position;
        step(s, ss->dseq, ss->S, 0, ss->K * ss->S, full, full ? &ss->sa : nullptr, position);
        s->prof_on = false;
        return;
    }
    if (!ss->use_graphs) {
        step(s, ss->dseq, ss->S, 0, ss->K * ss->S, full, full ? &ss->sa : nullptr, position);
        return;
    }
    hipGraphExec_t& g = (full ? ss->g_step : ss->g_body)[att_chunks(position) - 1];
    if (!g) g = capture(ss, full, position);
    HIP_OK(hipGraphLaunch(g, s->hs));
}

// Runs up to n more loop iterations (the first is the prefill), then waits for them.
int session_step(mgx_session* ss, int n) {
    mgx_stream* s = ss->s.get();
    HIP_OK(hipSetDevice(ss->m->device));
    const double t0 = now_s();
    const int first = ss->next;
    int done = 0;
    for (; done < n && ss->next < ss->S; ++done) {
        const int offset = ss->next++;
        const bool profiled = ss->prof_every > 0 && (offset - ss->start) % ss->prof_every == 0;
        if (offset == ss->start) {
            // prompt positions in groups, then the loop's first forward (one position at a time
            // through the captured body steps where a group cannot serve)
            if (!run_prefill(s, ss->dseq, ss->S, 0, ss->K * ss->S, 0, ss->start - 1))
                for (int pos = 0; pos < ss->start - 1; ++pos) run_position(ss, false, false, pos);
            run_position(ss, true, false, ss->start - 1);
            HIP_OK(hipGetLastError());
            HIP_OK(hipStreamSynchronize(s->hs));
            ss->prefill_seconds += now_s() - t0;
        } else {
            run_position(ss, true, profiled, offset - 1);
        }
    }
    HIP_OK(hipGetLastError());
    HIP_OK(hipStreamSynchronize(s->hs));
    if (done > 0) {
        // decode time excludes the prefill iteration, as report.decode_seconds does
        double el = now_s() - t0;
        if (first == ss->start) el -= ss->prefill_seconds;
        ss->decode_seconds += el;
    }
    s->used = ss->next > ss->start ? ss->next - 1 : 0;
    s->forwards = ss->next - ss->start;
    return done;
}

void session_finish(mgx_session* ss, int req, int32_t* codes_out, float* first_logits_out, float* step_logits_out,
                    mgx_generate_report* rep) {
    const mgx_lm_config& c = ss->m->c;
    mgx_stream* s = ss->s.get();
    const int K = ss->K, T = ss->T, S = ss->S;
    if (req < 0 || req >= ss->R) throw Error(MGX_ERR_INVALID, "request index out of range");
    if (rep) {
        rep->prefill_tokens = ss->start;
        rep->decode_steps = S - ss->start - 1;
        rep->forwards = ss->next - ss->start;
        rep->prefill_seconds = ss->prefill_seconds;
        rep->decode_seconds = ss->decode_seconds;
        rep->cache_bytes = mgx_stream_cache_bytes(s) / (uint64_t)ss->R;
    }
    const size_t per = (size_t)K * S;
    HIP_OK(hipMemcpy(ss->seq.data() + req * per, ss->dseq + req * per, per * 4, hipMemcpyDeviceToHost));
    if (first_logits_out && ss->next > ss->start)
        HIP_OK(hipMemcpy(first_logits_out, ss->dfirst + (size_t)req * K * c.card, sizeof(float) * (size_t)K * c.card,
                         hipMemcpyDeviceToHost));
    if (step_logits_out && ss->dsteps) {
        const size_t n = (size_t)(S - ss->start) * K * c.card;
        HIP_OK(hipMemcpy(step_logits_out, ss->dsteps + req * n, sizeof(float) * n, hipMemcpyDeviceToHost));
    }
    if (!codes_out) return;
    // revert_pattern_sequence + the final check (pipeline.cpp:307-313)
    const int32_t* seq = ss->seq.data() + req * per;
    for (size_t i = 0; i < (size_t)K * T; ++i) codes_out[i] = c.special_token_id;
    for (int q = 0; q < K; ++q)
        for (int st = 0; st < S; ++st) {
            const int t = ss->pattern_t(q, st);
            if (t >= 0) codes_out[(size_t)q * T + t] = seq[(size_t)q * S + st];
        }
    if (ss->next == S)
        for (size_t i = 0; i < (size_t)K * T; ++i)
            if (codes_out[i] < 0 || codes_out[i] >= c.card)
                throw Error(MGX_ERR_INVALID, "the generated sequence has a position the pattern never filled");
}

mgx_batch_request one_request(const float* t5_hidden, int32_t description_empty, const int32_t* prompt,
                              const mgx_generate_params* p) {
    if (!p) throw Error(MGX_ERR_INVALID, "null argument");
    mgx_batch_request r{};
    r.t5_hidden = t5_hidden; r.description_empty = description_empty; r.prompt_codes = prompt; r.params = *p;
    return r;
}

}  // namespace

extern "C" {

int mgx_session_create(mgx_model* m, const float* t5_hidden, int32_t n_ctx, int32_t description_empty,
                       const int32_t* prompt_codes, int32_t prompt_len, const mgx_generate_params* params,
                       int32_t keep_step_logits, mgx_session** out) {
    return guarded([&] {
        const mgx_batch_request r = one_request(t5_hidden, description_empty, prompt_codes, params);
        session_create(m, &r, 1, n_ctx, prompt_len, keep_step_logits, out);
    });
}

int mgx_session_step(mgx_session* ss, int32_t n_forwards, int32_t* done) {
    return guarded([&] {
        if (!ss) throw Error(MGX_ERR_INVALID, "null session");
        const int d = session_step(ss, n_forwards);
        if (done) *done = d;
    });
}

int32_t mgx_session_remaining(const mgx_session* ss) { return ss ? ss->S - ss->next : -1; }

int mgx_session_finish(mgx_session* ss, int32_t* codes_out, float* first_logits_out, float* step_logits_out,
                       mgx_generate_report* report) {
    return guarded([&] {
        if (!ss) throw Error(MGX_ERR_INVALID, "null session");
        session_finish(ss, 0, codes_out, first_logits_out, step_logits_out, report);
    });
}

int mgx_batch_create(mgx_model* m, const mgx_batch_request* requests, int32_t n_requests, int32_t n_ctx,
                     int32_t prompt_len, int32_t keep_step_logits, mgx_session** out) {
    return guarded([&] { session_create(m, requests, n_requests, n_ctx, prompt_len, keep_step_logits, out); });
}

int mgx_batch_finish(mgx_session* ss, int32_t request, int32_t* codes_out, float* first_logits_out,
                     float* step_logits_out, mgx_generate_report* report) {
    return guarded([&] {
        if (!ss) throw Error(MGX_ERR_INVALID, "null session");
        session_finish(ss, request, codes_out, first_logits_out, step_logits_out, report);
    });
}

int32_t mgx_session_requests(const mgx_session* ss) { return ss ? ss->R : -1; }

int mgx_session_profile(mgx_session* ss, int32_t every) {
    return guarded([&] {
        if (!ss) throw Error(MGX_ERR_INVALID, "null session");
        if (every < 0) throw Error(MGX_ERR_INVALID, "every must be >= 0");
        mgx_stream* s = ss->s.get();
        if (every > 0 && !s->stamps) {
            HIP_OK(hipSetDevice(ss->m->device));
            s->stamps = s->mem.alloc<unsigned long long>(2 * mgx::STAMP_SUB * (size_t)mgx_stream::STAMP_SLOTS);
            mgx::launch_stamp_init(s->stamps, mgx_stream::STAMP_SLOTS, s->hs);
            HIP_OK(hipGetLastError());
            int khz = 0;
            HIP_OK(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, ss->m->device));
            s->clock_khz = khz;
        }
        ss->prof_every = every;
    });
}

int mgx_session_profile_read(mgx_session* ss, int32_t kind, double* ms_total, double* bytes_total, int32_t* launches) {
    return guarded([&] {
        if (!ss) throw Error(MGX_ERR_INVALID, "null session");
        mgx_stream* s = ss->s.get();
        HIP_OK(hipStreamSynchronize(s->hs));
        double ms = 0.0, by = 0.0;
        int n = 0;
        if (!s->marks.empty()) {
            std::vector<unsigned long long> st(2 * mgx::STAMP_SUB * s->marks.size());
            HIP_OK(hipMemcpy(st.data(), s->stamps, st.size() * sizeof(unsigned long long), hipMemcpyDeviceToHost));
            for (const auto& mk : s->marks) {
                if (mk.kind != kind && mk.tag != kind) continue;
                unsigned long long b = ~0ull, e = 0ull;
                for (int k = 0; k < mgx::STAMP_SUB; ++k) {
                    b = std::min(b, st[2 * (mgx::STAMP_SUB * (size_t)mk.slot + k)]);
                    e = std::max(e, st[2 * (mgx::STAMP_SUB * (size_t)mk.slot + k) + 1]);
                }
                if (e <= b) continue;   // a launch that recorded nothing
                ms += (double)(e - b) / s->clock_khz; by += mk.bytes; ++n;
            }
        }
        if (ms_total) *ms_total = ms;
        if (bytes_total) *bytes_total = by;
        if (launches) *launches = n;
    });
}

void* mgx_session_hip_stream(mgx_session* ss) { return ss ? (void*)ss->s->hs : nullptr; }

void mgx_session_destroy(mgx_session* ss) { delete ss; }

int mgx_generate(mgx_model* m, const float* t5_hidden, int32_t n_ctx, int32_t description_empty,
                 const int32_t* prompt, int32_t prompt_len, const mgx_generate_params* p,
                 int32_t* codes_out, float* first_logits_out, float* step_logits_out, mgx_generate_report* rep) {
    return guarded([&] {
        if (!codes_out || !rep) throw Error(MGX_ERR_INVALID, "null argument");
        mgx_session* raw = nullptr;
        const mgx_batch_request r = one_request(t5_hidden, description_empty, prompt, p);
        session_create(m, &r, 1, n_ctx, prompt_len, step_logits_out != nullptr, &raw);
        std::unique_ptr<mgx_session> ss(raw);
        session_step(ss.get(), ss->S);
        session_finish(ss.get(), 0, codes_out, first_logits_out, step_logits_out, rep);
    });
}

}  // extern "C"

// ------------------------------------------------------------------------------------
// slotted batches: the server's device side (library-internal, declared in slots.h)
// ------------------------------------------------------------------------------------
// `n` slots of `cpr` streams (2: guided or not, 1: unguided only) share one stream of n * cpr
// columns. A request is opened into a free slot between steps: its delay-pattern sequence,
// mask and uniforms go to the slot's rows, its conditioning to the slot's cross K / V, its
// prompt before the last position runs through the prefill view aimed at the slot (slot_prefill)
// and its position goes to start - 1 (0 for a prompt too short for a group). Every step then
// processes each live slot's next position -- any prompt positions left (no sampling), then
// its loop offsets start..S-1 (sampling) -- and the device
// retires a slot after its last offset (k_advance). Each request computes exactly what it
// computes alone: every column's arithmetic depends only on that column's inputs.
struct mgx_slots {
    mgx_model* m = nullptr;
    std::unique_ptr<mgx_stream> s;
    DevArena mem;
    int n = 0, cpr = 1, K = 0, seq_len = 0, max_gen = 0, max_ctx = 0, step_rows = 0;
    int32_t* dseq = nullptr;       // [n][K][seq_len]
    uint8_t* dmask = nullptr;      // [n][K][seq_len]
    float* duni = nullptr;         // [n][seq_len][K]
    float *dfirst = nullptr, *dsteps = nullptr;
    // pinned staging, one region per slot: a slot's region is reused only after its previous
    // request's results were read, which waits for the stream
    int32_t* hseq = nullptr;
    uint8_t* hmask = nullptr;
    float *huni = nullptr, *ht5 = nullptr;
    mgx::SampleArgs sa{};
    hipGraphExec_t g[mgx::ATT_MAX_CHUNKS] = {};
    bool use_graphs = true;
    struct Slot { bool live = false, unread = false; int pos = 0, start = 0, S = 0, T = 0; };
    std::vector<Slot> slot;
    ~mgx_slots() {
        if (s && s->hs) (void)hipStreamSynchronize(s->hs);
        for (auto& e : g)
            if (e) (void)hipGraphExecDestroy(e);
        for (void* p : {(void*)hseq, (void*)hmask, (void*)huni, (void*)ht5})
            if (p) (void)hipHostFree(p);
        mem.release();
    }
};

namespace {

template <typename T> T* host_alloc(size_t count) {
    void* p = nullptr;
    HIP_OK(hipHostMalloc(&p, std::max<size_t>(count, 1) * sizeof(T), hipHostMallocDefault));
    return (T*)p;
}

void slots_create(mgx_model* m, int n, int cpr, int max_gen, int max_ctx, int keep_steps, mgx_slots** out) {
    if (!m || !out) throw Error(MGX_ERR_INVALID, "null argument");
    *out = nullptr;
    const mgx_lm_config& c = m->c;
    if (cpr != 1 && cpr != 2) throw Error(MGX_ERR_INVALID, "streams per slot must be 1 or 2");
    if (n <= 0 || n * cpr > 16) throw Error(MGX_ERR_INVALID, "at most 16 streams (8 slots of 2)");
    if (max_gen <= 0) throw Error(MGX_ERR_INVALID, "max_gen_len must be positive");
    if (max_ctx <= 0 || max_ctx > 256) throw Error(MGX_ERR_INVALID, "the conditioning limit must be 1 to 256 tokens");
    auto sl = std::make_unique<mgx_slots>();
    sl->m = m; sl->n = n; sl->cpr = cpr; sl->K = c.n_q; sl->max_gen = max_gen; sl->max_ctx = max_ctx;
    sl->seq_len = 1 + max_gen + (c.n_q - 1);
    if (const char* g = std::getenv("MGX_GRAPHS")) sl->use_graphs = std::strcmp(g, "0") != 0;
    mgx_stream* raw = nullptr;
    make_stream(m, sl->seq_len, n * cpr, n, nullptr, max_ctx, cpr == 2 ? 1 : 0, &raw);
    sl->s.reset(raw);
    mgx_stream* st = sl->s.get();
    const size_t per = (size_t)sl->K * sl->seq_len;
    st->dlive = st->mem.alloc<int>((size_t)n);
    st->dpar = st->mem.alloc<mgx::ReqParams>((size_t)n);
    st->dnc = st->mem.alloc<int>((size_t)n);
    HIP_OK(hipMemsetAsync(st->dlive, 0, sizeof(int) * n, st->hs));
    HIP_OK(hipMemsetAsync(st->dpar, 0, sizeof(mgx::ReqParams) * n, st->hs));
    HIP_OK(hipMemsetAsync(st->dnc, 0, sizeof(int) * n, st->hs));
    sl->dseq = sl->mem.alloc<int32_t>(per * n);
    sl->dmask = sl->mem.alloc<uint8_t>(per * n);
    sl->duni = sl->mem.alloc<float>(per * n);
    sl->dfirst = sl->mem.alloc<float>((size_t)n * sl->K * c.card);
    // an idle slot embeds its row 0: keep it a valid id
    std::vector<int32_t> init(per * n, c.special_token_id);
    HIP_OK(hipMemcpy(sl->dseq, init.data(), init.size() * 4, hipMemcpyHostToDevice));
    HIP_OK(hipMemsetAsync(sl->dmask, 0, per * n, st->hs));
    HIP_OK(hipMemsetAsync(sl->duni, 0, per * n * sizeof(float), st->hs));
    sl->step_rows = sl->seq_len - 1;
    if (keep_steps) sl->dsteps = sl->mem.alloc<float>((size_t)n * sl->step_rows * sl->K * c.card);
    sl->hseq = host_alloc<int32_t>(per * n);
    sl->hmask = host_alloc<uint8_t>(per * n);
    sl->huni = host_alloc<float>(per * n);
    if (cpr == 2) sl->ht5 = host_alloc<float>((size_t)n * max_ctx * c.cond_dim);
    mgx::SampleArgs& sa = sl->sa;
    sa.logits = st->logits; sa.n_q = sl->K; sa.card = c.card; sa.n_req = n; sa.cpr = cpr; sa.par = st->dpar;
    sa.pos = st->dpos; sa.live = st->dlive; sa.seq_len = sl->seq_len; sa.mask = sl->dmask; sa.mask_stride = (long long)per;
    sa.special = c.special_token_id; sa.uniforms = sl->duni; sa.seq = sl->dseq;
    sa.first_logits = sl->dfirst; sa.step_logits = sl->dsteps; sa.step_rows = sl->step_rows;
    sl->slot.assign((size_t)n, mgx_slots::Slot{});
    HIP_OK(hipStreamSynchronize(st->hs));
    *out = sl.release();
}

// The checks a request passes before it may wait for a slot (no device work).
void slot_check(const mgx_slots* sl, const mgx_batch_request& q, int n_ctx, int prompt_len) {
    if (!sl) throw Error(MGX_ERR_INVALID, "null argument");
    check_request(sl->m->c, q, n_ctx, prompt_len);
    if (q.params.max_gen_len > sl->max_gen) throw Error(MGX_ERR_INVALID, "max_gen_len above the server's limit");
    const bool guided = mgx_use_guidance(q.params.cfg_coef, q.description_empty) != 0;
    if (guided && sl->cpr != 2) throw Error(MGX_ERR_INVALID, "a guided request needs slots of two streams");
    if (guided && n_ctx > sl->max_ctx) throw Error(MGX_ERR_INVALID, "conditioning longer than the server's limit");
    if (guided && !q.t5_hidden) throw Error(MGX_ERR_INVALID, "the conditioning has no tokens");
}

// Runs positions 0 .. count - 1 of slot r (its prompt before the last position) through the
// slots stream's prefill view aimed at the slot, prefill_positions at a time, and moves the
// slot's device position to count. The same columns as batch steps would compute (each at its
// own position, causal by key count), so the slot's caches hold the same values. Returns false,
// running nothing, when the prompt is too short for a group or the view cannot serve the slots.
bool slot_prefill(mgx_slots* sl, int r, int count, int nc) {
    mgx_stream* st = sl->s.get();
    if (count < 2 || st->cpr > 8 || (st->cpr & (st->cpr - 1))) return false;
    if (!st->pf) st->pf = make_prefill_view(st, prefill_positions(st));
    mgx_stream* pf = st->pf.get();
    aim_view(pf, st, r);
    const int G = pf->n_req;
    if (pf->dnc) mgx::launch_fill_i32(pf->dnc, G, nc, st->hs);
    const int32_t* ids = sl->dseq + (size_t)r * sl->K * sl->seq_len;
    for (int p0 = 0; p0 < count; p0 += G) {
        const int g = std::min(G, count - p0);
        mgx::launch_set_positions(pf->dpos, g, p0, st->hs);
        step(pf, ids, sl->seq_len, 0, 0, false, nullptr, p0 + g - 1, g * pf->cpr);
    }
    mgx::launch_set_positions(st->dpos + r, 1, count, st->hs);
    return true;
}

void slot_open(mgx_slots* sl, int r, const mgx_batch_request& q, int n_ctx, int prompt_len) {
    slot_check(sl, q, n_ctx, prompt_len);
    if (r < 0 || r >= sl->n) throw Error(MGX_ERR_INVALID, "slot index out of range");
    mgx_slots::Slot& h = sl->slot[(size_t)r];
    if (h.live || h.unread) throw Error(MGX_ERR_STATE, "the slot is in use");
    const mgx_lm_config& c = sl->m->c;
    mgx_stream* st = sl->s.get();
    HIP_OK(hipSetDevice(sl->m->device));
    const int K = sl->K, L = sl->seq_len, T = q.params.max_gen_len, S = 1 + T + (K - 1), start = prompt_len + 1;
    const bool guided = mgx_use_guidance(q.params.cfg_coef, q.description_empty) != 0;
    const size_t per = (size_t)K * L;
    int32_t* seq = sl->hseq + per * r;
    uint8_t* mask = sl->hmask + per * r;
    float* uni = sl->huni + per * r;
    // the delay pattern of mg_generate (pattern.h:31-115): timestep t = st - 1 - q, S = T + n_q
    const auto pat = [T](int qq, int stp) { const int t = stp - 1 - qq; return (stp > 0 && t >= 0 && t < T) ? t : -1; };
    for (int qq = 0; qq < K; ++qq)
        for (int stp = 0; stp < L; ++stp) {
            const int t = stp < S ? pat(qq, stp) : -1;
            mask[(size_t)qq * L + stp] = t >= 0;
            seq[(size_t)qq * L + stp] =
                t < 0 ? c.special_token_id : (t < prompt_len ? q.prompt_codes[(size_t)qq * prompt_len + t] : -1);
        }
    std::fill(uni, uni + per, 0.0f);
    const mgx_generate_params& p = q.params;
    if (p.use_sampling && p.temperature > 0.0f) {
        std::mt19937 g((uint32_t)p.seed);
        for (int stp = start; stp < S; ++stp)
            for (int qq = 0; qq < K; ++qq)
                if (mask[(size_t)qq * L + stp]) uni[(size_t)stp * K + qq] = ((g() >> 8) + 0.5f) * (1.0f / 16777216.0f);
    }
    HIP_OK(hipMemcpyAsync(sl->dseq + per * r, seq, per * 4, hipMemcpyHostToDevice, st->hs));
    HIP_OK(hipMemcpyAsync(sl->dmask + per * r, mask, per, hipMemcpyHostToDevice, st->hs));
    HIP_OK(hipMemcpyAsync(sl->duni + per * r, uni, per * 4, hipMemcpyHostToDevice, st->hs));
    if (guided) {
        float* t5 = sl->ht5 + (size_t)r * sl->max_ctx * c.cond_dim;
        std::memcpy(t5, q.t5_hidden, sizeof(float) * (size_t)n_ctx * c.cond_dim);
        project_memory(st, r, t5, n_ctx);
    }
    mgx::launch_slot_open(st->dpos, st->dlive, st->dpar, st->dnc, r, req_params(p, guided, start, S),
                          guided ? n_ctx : 0, st->hs);
    // the prompt before its last position in groups (no sampling happens there)
    const int pre = slot_prefill(sl, r, start - 1, guided ? n_ctx : 0) ? start - 1 : 0;
    HIP_OK(hipGetLastError());
    h.live = true; h.unread = true; h.pos = pre; h.start = start; h.S = S; h.T = T;
}

hipGraphExec_t slots_capture(mgx_slots* sl, int position) {
    mgx_stream* s = sl->s.get();
    hipGraph_t g = nullptr;
    hipGraphExec_t e = nullptr;
    HIP_OK(hipStreamBeginCapture(s->hs, hipStreamCaptureModeThreadLocal));
    step(s, sl->dseq, sl->seq_len, 0, sl->K * sl->seq_len, true, &sl->sa, position);
    HIP_OK(hipStreamEndCapture(s->hs, &g));
    const hipError_t rc = hipGraphInstantiate(&e, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    HIP_OK(rc);
    return e;
}

// Enqueues `steps` batch steps (no wait). The host mirrors every slot's position: the device
// advances and retires live slots by the same rule (k_advance).
void slots_run(mgx_slots* sl, int steps) {
    mgx_stream* s = sl->s.get();
    HIP_OK(hipSetDevice(sl->m->device));
    for (int i = 0; i < steps; ++i) {
        int top = 0;
        for (const auto& h : sl->slot)
            if (h.live) top = std::max(top, h.pos);
        if (!sl->use_graphs) {
            step(s, sl->dseq, sl->seq_len, 0, sl->K * sl->seq_len, true, &sl->sa, top);
        } else {
            hipGraphExec_t& g = sl->g[att_chunks(top) - 1];
            if (!g) g = slots_capture(sl, top);
            HIP_OK(hipGraphLaunch(g, s->hs));
        }
        for (auto& h : sl->slot)
            if (h.live) {
                if (h.pos + 2 >= h.S) { h.live = false; h.pos = 0; }
                else ++h.pos;
            }
    }
    HIP_OK(hipGetLastError());
}

// A retired slot's results (waits for the stream): codes reverted as mg_generate returns them.
void slot_read(mgx_slots* sl, int r, int32_t* codes_out, float* first_out, float* steps_out) {
    if (r < 0 || r >= sl->n) throw Error(MGX_ERR_INVALID, "slot index out of range");
    mgx_slots::Slot& h = sl->slot[(size_t)r];
    if (h.live || !h.unread) throw Error(MGX_ERR_STATE, "the slot holds no finished request");
    const mgx_lm_config& c = sl->m->c;
    mgx_stream* st = sl->s.get();
    HIP_OK(hipSetDevice(sl->m->device));
    HIP_OK(hipStreamSynchronize(st->hs));
    const int K = sl->K, L = sl->seq_len, T = h.T, S = h.S;
    const size_t per = (size_t)K * L;
    int32_t* seq = sl->hseq + per * r;
    HIP_OK(hipMemcpy(seq, sl->dseq + per * r, per * 4, hipMemcpyDeviceToHost));
    if (first_out)
        HIP_OK(hipMemcpy(first_out, sl->dfirst + (size_t)r * K * c.card, sizeof(float) * K * c.card,
                         hipMemcpyDeviceToHost));
    if (steps_out) {
        if (!sl->dsteps) throw Error(MGX_ERR_STATE, "per-step logits were not kept");
        HIP_OK(hipMemcpy(steps_out, sl->dsteps + (size_t)r * sl->step_rows * K * c.card,
                         sizeof(float) * (size_t)(S - h.start) * K * c.card, hipMemcpyDeviceToHost));
    }
    h.unread = false;
    if (!codes_out) return;
    // revert_pattern_sequence + the final check (pipeline.cpp:307-313)
    for (size_t i = 0; i < (size_t)K * T; ++i) codes_out[i] = c.special_token_id;
    for (int q = 0; q < K; ++q)
        for (int stp = 0; stp < S; ++stp) {
            const int t = stp - 1 - q;
            if (stp > 0 && t >= 0 && t < T) codes_out[(size_t)q * T + t] = seq[(size_t)q * L + stp];
        }
    for (size_t i = 0; i < (size_t)K * T; ++i)
        if (codes_out[i] < 0 || codes_out[i] >= c.card)
            throw Error(MGX_ERR_INVALID, "the generated sequence has a position the pattern never filled");
}

}  // namespace

#include "slots.h"

int mgx_internal_slots_create(mgx_model* m, int n, int cpr, int max_gen, int max_ctx, int keep_steps, mgx_slots** out) {
    return guarded([&] { slots_create(m, n, cpr, max_gen, max_ctx, keep_steps, out); });
}
int mgx_internal_slot_check(const mgx_slots* sl, const mgx_batch_request* q, int n_ctx, int prompt_len) {
    return guarded([&] {
        if (!q) throw Error(MGX_ERR_INVALID, "null argument");
        slot_check(sl, *q, n_ctx, prompt_len);
    });
}
int mgx_internal_slot_open(mgx_slots* sl, int r, const mgx_batch_request* q, int n_ctx, int prompt_len) {
    return guarded([&] {
        if (!q) throw Error(MGX_ERR_INVALID, "null argument");
        slot_open(sl, r, *q, n_ctx, prompt_len);
    });
}
int mgx_internal_slots_run(mgx_slots* sl, int steps) { return guarded([&] { slots_run(sl, steps); }); }
int mgx_internal_slots_sync(mgx_slots* sl) {
    return guarded([&] {
        HIP_OK(hipSetDevice(sl->m->device));
        HIP_OK(hipStreamSynchronize(sl->s->hs));
    });
}
int mgx_internal_slot_read(mgx_slots* sl, int r, int32_t* codes_out, float* first_out, float* steps_out) {
    return guarded([&] { slot_read(sl, r, codes_out, first_out, steps_out); });
}
void mgx_internal_slot_state(const mgx_slots* sl, int r, int* live, int* pos, int* start, int* S) {
    const mgx_slots::Slot& h = sl->slot[(size_t)r];
    *live = h.live; *pos = h.pos; *start = h.start; *S = h.S;
}
uint64_t mgx_internal_slot_cache_bytes(const mgx_slots* sl) { return mgx_stream_cache_bytes(sl->s.get()) / sl->n; }
void mgx_internal_slots_destroy(mgx_slots* sl) { delete sl; }
