// kernels.h -- argument blocks and launchers of the decode-step kernels (kernels.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mgx {

enum { T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q8_0 = 8 };
enum { ACT_Q8 = 0, ACT_F16 = 1, ACT_F32 = 2 };
// GEMV prologues: LayerNorm of f32 columns, plain conversion of f32 columns, or a copy of
// columns already in activation form -- all into LDS, while the weight loads are in flight.
enum { PRO_LN = 0, PRO_F32 = 1, PRO_ACT = 2 };
// GEMV epilogues: store, residual add, q + KV-cache append, GELU then activation form.
enum { EPI_STORE = 0, EPI_RESID = 1, EPI_QKV = 2, EPI_GELU_ACT = 3 };

constexpr int ATT_CHUNK = 256;   // keys per attention chunk (fixes the reduction order)
constexpr int ATT_MAX_CHUNKS = 16;  // capacity up to 4096 positions
constexpr int ATT_SUB = 64;         // keys per score block
constexpr int ATT_SUBS = ATT_CHUNK / ATT_SUB;
constexpr int MAX_CARD = 2048;   // sampler's LDS rows

// A weight matrix in device layout: `out` rows of `in`. Q8_0: int8 q[out][in] + fp16
// d[out][in/32]; Q4_0: the 16 nibble bytes of each block q[out][in/2] + d; F16 / F32: q only.
struct DevMat {
    int type, in, out;
    const void* q;
    const uint16_t* d;
};

// Activation columns in the form the consuming weights multiply against.
struct ActBuf {
    int kind;      // ACT_Q8 / ACT_F16 / ACT_F32
    int stride;    // elements per column
    int8_t* q;     // Q8 quants [col][stride]
    float* d;      // Q8 scales [col][stride/32] (fp16 values widened)
    uint16_t* h;   // fp16 [col][stride]
    float* f;      // f32 [col][stride]
};

struct EmbedArgs {
    DevMat emb[8];
    int n_q;
    const int32_t* ids;   // codebook q's token for position p at ids[q * ids_stride + p - ids_base]
    int ids_stride, ids_base;
    const float* table;   // sinusoid [capacity][dim]
    const int* pos;       // device position of this step
    int dim;
    float* x;             // [ncol][dim]
    int ncol;
};

struct GemvArgs {
    DevMat w;
    int ncol;
    int pro;
    const float* x;       // PRO_LN / PRO_F32 source [col][x_stride]
    int x_stride;
    const float *ln_w, *ln_b;
    float eps;
    ActBuf src;           // PRO_ACT source
    int epi;
    float* y;             // STORE / RESID: [col][y_stride]; QKV: q [col][dim]
    int y_stride;
    float *k, *v;         // QKV: caches [col][heads][cap][64]
    int dim, heads, cap;
    const int* pos;       // QKV: device position
    ActBuf dst;           // GELU_ACT destination
    unsigned long long* stamp;   // optional [64][2]: per-sub-slot earliest start, latest end (GPU wall clock)
};

struct AttnArgs {
    const float* q;       // [col][dim]
    const float* k;       // [col][heads][cap][64]
    const float* v;       // [col][heads][cap][64]
    float* scores;        // [col][heads][cap]
    float* opart;         // [col][heads][max_chunks][64]
    float* cmax;          // [col][heads][max_chunks * ATT_SUBS] score-block maxima
    int dim, heads, cap, max_chunks, ncol;
    float scale;
    const int* pos;       // device position: keys [0, pos]
    ActBuf out;           // the out-projection's activation
    unsigned long long* stamp;   // optional [64][2]: scores' earliest starts, reduce's latest ends
};

struct XAttnArgs {
    const float* q;   // [dim]
    const float* k;   // [heads][n_ctx][64]
    const float* v;
    int n_ctx;
    float scale;
    ActBuf out;       // column 0 of cross.out's activation
};

struct SampleArgs {
    const float* logits;     // [n_seq][n_q][card]
    int n_q, card, guided;
    float cfg_coef;
    const uint8_t* mask;     // [n_q][steps]
    int steps, start;
    const int* pos;          // the loop offset is *pos + 1
    int use_sampling;
    float temperature;
    int top_k;
    const float* uniforms;   // [steps][n_q]
    int special;
    int32_t* seq;            // [n_q][steps]
    float* first_logits;     // [n_q][card], written at offset == start
    float* step_logits;      // [steps - start][n_q][card] or null
};

void launch_embed(const EmbedArgs& a, hipStream_t s);
void launch_gemv(const GemvArgs& a, hipStream_t s);
// nch: the 256-key chunks of the position the launch runs at (the grid covers exactly these)
void launch_attention(const AttnArgs& a, int nch, hipStream_t s);
void launch_xattn(const XAttnArgs& a, int heads, hipStream_t s);
void launch_add_bias(float* y, const float* b, int n, int ncol, hipStream_t s);
void launch_xkv_split(const float* kv, int n_ctx, int dim, float* k, float* v, hipStream_t s);
void launch_sample(const SampleArgs& a, hipStream_t s);
void launch_advance(int* pos, hipStream_t s);
// fills n launch-timing slots (64 sub-slots each) with {UINT64_MAX, 0}
void launch_stamp_init(unsigned long long* p, int n, hipStream_t s);
void launch_repack(int type, const uint8_t* raw, int64_t rows, int in, void* q, uint16_t* d, hipStream_t s);

}  // namespace mgx
