// kernels.h -- argument blocks and launchers of the decode-step kernels (kernels.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mgx {

enum { T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q8_0 = 8 };
enum { ACT_Q8 = 0, ACT_F16 = 1, ACT_F32 = 2 };
enum { EPI_STORE = 0, EPI_RESID = 1, EPI_GELU = 2, EPI_QKV = 3 };

constexpr int ATT_CHUNK = 256;   // keys per attention chunk (fixes the reduction order)
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
    const int32_t* ids;
    int ids_stride;    // ids of codebook q at ids[q * ids_stride]
    const float* pos;  // [capacity][dim]
    int position;
    int dim;
    float* x;          // [ncol][dim]
    int ncol;
};

struct LnArgs {
    const float* x;
    int x_stride, dim;
    const float *w, *b;
    float eps;
    ActBuf out;
};

struct ActArgs {
    const float* x;
    int x_stride, n;
    ActBuf out;
};

struct GemvOut {
    int mode;
    float* y;        // STORE / GELU: y[col][y_stride]; RESID: y += ; QKV: q [col][dim]
    int y_stride;
    float *k, *v;    // QKV: caches [col][heads][cap][64]
    int dim, heads, cap, position;
};

struct GemvArgs {
    DevMat w;
    ActBuf act;
    int ncol;
    GemvOut o;
};

struct AttnArgs {
    const float* q;   // [col][dim]
    const float* k;   // [col][heads][cap][64]
    const float* v;   // [col][heads][cap][64]
    float* scores;    // [col][heads][cap]
    float* opart;     // [col][heads][max_chunks][64]
    int dim, heads, cap, position, max_chunks, ncol;
    float scale;
};

struct XAttnArgs {
    const float* q;   // [dim]
    const float* k;   // [heads][n_ctx][64]
    const float* v;
    float* o;         // [dim]
    int n_ctx;
    float scale;
};

struct SampleArgs {
    const float* logits;     // [n_seq][n_q][card]
    int n_q, card, guided;
    float cfg_coef;
    const uint8_t* mask;     // [n_q][steps]
    int steps, offset;
    int use_sampling;
    float temperature;
    int top_k;
    const float* uniforms;   // [steps][n_q]
    int special;
    int32_t* seq;            // [n_q][steps]
    float* first_logits;     // [n_q][card] or null
    float* step_logits;      // [n_q][card] or null
};

void launch_embed(const EmbedArgs& a, hipStream_t s);
void launch_ln_act(const LnArgs& a, int ncol, hipStream_t s);
void launch_act(const ActArgs& a, int ncol, hipStream_t s);
void launch_add_bias(float* y, const float* b, int n, int ncol, hipStream_t s);
void launch_gemv(const GemvArgs& a, hipStream_t s);
void launch_attention(const AttnArgs& a, const ActBuf& out, hipStream_t s);
void launch_xattn(const XAttnArgs& a, int heads, hipStream_t s);
void launch_xkv_split(const float* kv, int n_ctx, int dim, float* k, float* v, hipStream_t s);
void launch_sample(const SampleArgs& a, hipStream_t s);
void launch_repack(int type, const uint8_t* raw, int64_t rows, int in, void* q, uint16_t* d, hipStream_t s);

}  // namespace mgx
