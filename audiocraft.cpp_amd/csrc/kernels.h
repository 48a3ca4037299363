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

constexpr int ATT_CHUNK = 64;       // keys per attention chunk (fixes the reduction order)
constexpr int ATT_SPAN = 256;       // cache rows per head are allocated in whole 256-key spans; a
                                    // step's attention grid covers the 64-key chunks of its key count
constexpr int ATT_MAX_SPANS = 16;   // capacity up to 4096 positions
constexpr int ATT_MAX_CHUNKS = ATT_MAX_SPANS * ATT_SPAN / ATT_CHUNK;
constexpr int ATT_PF_WAVES = 4;   // prefill attention: waves per block, two query columns per
constexpr int ATT_PF_PASSES = 4;  // wave and pass, all sharing one staged chunk's K / V in LDS
constexpr int ATT_PF_COLS = 2 * ATT_PF_WAVES * ATT_PF_PASSES;
constexpr int MAX_CARD = 2048;   // sampler's LDS rows
constexpr int STAMP_SUB = 256;   // sub-slots of a profiled launch's timing slot
constexpr int MF_MAX_COLS = 512;   // matrix-core GEMV columns per launch (16-column groups): a prefill group
constexpr int MF_WIDE_GROUPS = 8;  // column groups one wide matrix-core block holds at most

// A weight matrix in device layout: `out` rows of `in`. Q8_0: int8 q[out][in] + fp16
// d[out][in/32]; Q4_0: the 16 nibble bytes of each block q[out][in/2] + d; F16 / F32: q only.
// For the matrix-core GEMV (Q8_0 and Q4_0, or null): dt, the scales tile-transposed
// [out/16][in/32][16]; qm, the quants again in operand order [out/16][in/32][64 lanes][8 or 4
// bytes]: lane 16g + c holds row 16 * tile + c, elements 8g..8g+7 of the block (Q4_0: byte m
// holds element 8g + m in its low nibble and 8g + m + 4 in its high one).
struct DevMat {
    int type, in, out;
    const void* q;
    const uint16_t* d;
    const uint16_t* dt;
    const int8_t* qm;
};

// Activation columns in the form the consuming weights multiply against.
struct ActBuf {
    int kind;      // ACT_Q8 / ACT_F16 / ACT_F32
    int stride;    // elements per column
    int8_t* q;     // Q8 quants [col][stride]; block-major: [stride/32][4 g][16 col][8], element
                   // 32b + 8g + j of column c at (b * 64 + 16g + c) * 8 + j (matrix-core operand order)
    float* d;      // Q8 scales [col][stride/32] (fp16 values widened); block-major: [stride/32][16 col]
    uint16_t* h;   // fp16 [col][stride]
    float* f;      // f32 [col][stride]
    int bm;        // Q8 block-major (the matrix-core GEMV's source; at most 16 columns)
};

struct EmbedArgs {
    DevMat emb[8];
    int n_q;
    const int32_t* ids;   // codebook q's token for position p at ids[q * ids_stride + p - ids_base]
    int ids_stride, ids_base;
    int ids_req_stride, cols_per_req;   // column n reads request n / cols_per_req's ids (+ that * ids_req_stride)
    const float* table;   // sinusoid [capacity][dim]
    const int* pos;       // [request] device position of this step
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
    const int* pos;       // QKV: [request] device positions; column n belongs to request n >> cshift
    int cshift;
    int kv_cols;          // QKV: 0, or the cache column count when columns share caches (column n -> n % kv_cols)
    ActBuf dst;           // GELU_ACT destination
    float* dst_f;         // GELU_ACT: optional f32 copy [col][dst.stride] (an adapted consumer's A x reads it)
    // optional adapter on this projection (lora.h:50-83): y = Wx + s*B(Ax), DoRA rows scale
    // y by m / ||W + sBA||, then the strength blend; applied before the epilogue
    const float* ad_ax;   // [col][ad_rank] A x of the launch's columns; null = no adapter
    const float* ad_B;    // [out][ad_rank]
    const float* ad_m;    // [out] magnitude (DoRA) or null (plain LoRA)
    const float* ad_norm; // [out] ||W + sBA|| per row (DoRA)
    int ad_rank;
    float ad_scale, ad_strength;
    // optional per-column gate (STORE / RESID): columns whose gate is 0 keep their destination
    const int* gate;
    int col0;             // the launch's first column in the caller's numbering (pos, gate)
    int stream_w;         // vector GEMV: 1 when this launch is the only one reading the weights
                          // this step (non-temporal loads), 0 when column pairs re-read them
    int ygroups;          // vector GEMV: > 1 when blockIdx.y runs that many whole groups of the
                          // launch's ncol columns, group g at column g * ncol of the arguments
    unsigned long long* stamp;   // optional [STAMP_SUB][2]: per-sub-slot earliest start, latest end (GPU wall clock)
};

struct AttnArgs {
    const float* q;       // [col][dim]
    const float* k;       // [col][heads][cap][64]
    const float* v;       // [col][heads][cap][64]
    float* opart;         // [col][heads][max_chunks][64] each chunk's V.e
    float* cmax;          // [col][heads][max_chunks] each chunk's score max
    double* csum;         // [col][heads][max_chunks] each chunk's sum of e
    int dim, heads, cap, max_chunks, ncol;
    float scale;
    const int* pos;       // [request] device positions: column n attends keys [0, pos[n >> cshift]]
    int cshift;
    int kv_cols;          // 0, or the cache column count when columns share caches (column n -> n % kv_cols)
    int nch;              // set by launch_attention: the launch's chunk count
    ActBuf out;           // the out-projection's activation
    float* out_f;         // optional f32 copy [col][dim] (an adapted out-projection's A x reads it)
    unsigned long long* stamp;   // optional [STAMP_SUB][2]: the chunk kernel's earliest starts, the combine's latest ends
};

// One block per (head, request r): q + r*dim, k / v + r*heads*n_ctx*64, output column r.
struct XAttnArgs {
    const float* q;   // [n_req][dim]
    const float* k;   // [n_req][heads][n_ctx][64]
    const float* v;
    int n_ctx, dim;   // n_ctx: the rows per head (every request's count when nc is null)
    const int* nc;    // optional [n_req] conditioning tokens per request (0: writes zeros)
    // optional additive score bias: query r of head h adds bias[(h * n_req + r) * bias_stride + key]
    const float* bias;
    int bias_stride;
    int shared_kv;    // every query attends the same keys (k, v of request 0)
    float scale;
    ActBuf out;       // cross.out's activation, column r
    float* out_f;     // optional f32 copy [n_req][dim]
    unsigned long long* stamp;   // optional [STAMP_SUB][2]: the launch's earliest block start, latest end
};

constexpr int MAX_REQ = 16;      // requests of one batched session

// A request's sampling parameters and loop bounds, in device memory (one per request) so that
// a captured step serves whichever requests a batch holds.
struct ReqParams {
    float cfg_coef, temperature;
    int use_sampling, top_k, guided;
    int start, steps;   // the loop runs offsets start .. steps - 1 (pipeline.cpp:255-302)
    int pad;
};

// One block per (codebook, request). Request r samples at offset pos[r] + 1 when that offset
// is in [start, steps) and, with `live` set, live[r] != 0.
struct SampleArgs {
    const float* logits;     // [n_req][cpr][n_q][card]: column 0 conditional, column 1 null
    int n_q, card, n_req, cpr;
    const ReqParams* par;    // [n_req]
    const int* pos;          // [n_req]
    const int* live;         // [n_req] or null (every request)
    int seq_len;             // row length of mask, uniforms and seq
    const uint8_t* mask;     // request r's at mask + r * mask_stride: [n_q][seq_len]
    long long mask_stride;   // 0: one delay pattern for every request
    int special;
    const float* uniforms;   // [n_req][seq_len][n_q]
    int32_t* seq;            // [n_req][n_q][seq_len]
    float* first_logits;     // [n_req][n_q][card], written at offset == start
    float* step_logits;      // [n_req][step_rows][n_q][card] (row offset - start) or null
    int step_rows;
};

void launch_embed(const EmbedArgs& a, hipStream_t s);
// A GEMV launch (the matrix-core kernel when gemv_mf_ok, otherwise the vector kernels in groups
// of two columns).
void launch_gemv(const GemvArgs& a, hipStream_t s);
// True when launch_gemv runs `a` on the matrix cores: Q8_0 weights with dt and qm, 3 to 16
// columns, a supported width, rows a multiple of the tile, a PRO_ACT source in block-major Q8.
bool gemv_mf_ok(const GemvArgs& a);
// Q8 activation columns from f32 ones for a matrix-core GEMV: a.x / x_stride (+ LayerNorm
// a.ln_w / ln_b / eps when a.pro == PRO_LN) -> a.dst (block-major Q8, stride a.w.in), exactly as
// the vector GEMV's prologue builds them; a.ncol columns. With a.w.q set (an adapter's A, f32
// [rank][in]) it also writes A x of the same columns to a.y [col][a.y_stride].
void launch_act_prep(const GemvArgs& a, hipStream_t s);
// dt from d, and qm from q, for a Q8_0 matrix (out a multiple of 16)
void launch_scales_t(const DevMat& w, uint16_t* dt, hipStream_t s);
void launch_weights_mf(const DevMat& w, int8_t* qm, hipStream_t s);
// the Q4_0 operand-order copy (one word of 8 nibbles per lane and block) for a Q4_0 matrix
void launch_weights_mf4(const DevMat& w, uint32_t* qm, hipStream_t s);
// Self-attention in two launches: one block per (64-key chunk, head, column) for the chunk's
// max, sum and V.e, then one wave per (head, column) combining the chunks. nch: the chunks the
// grid covers (at least those of the largest position in the launch; a block past its column's
// position exits at once).
void launch_attention(const AttnArgs& a, int nch, hipStream_t s);
void launch_xattn(const XAttnArgs& a, int heads, int n_req, hipStream_t s);
void launch_add_bias(float* y, const float* b, int n, int ncol, hipStream_t s);
// rows: the row count per head of k and v (>= n_ctx)
void launch_xkv_split(const float* kv, int n_ctx, int rows, int dim, float* k, float* v, hipStream_t s);
void launch_sample(const SampleArgs& a, hipStream_t s);
// The position step after a forward: with live null every request's position advances; with
// live set only live requests advance, and one whose next offset would reach par.steps
// retires (live 0, position 0).
void launch_advance(int* pos, int* live, const ReqParams* par, int n_req, hipStream_t s);
// pos[r] = p0 + r for r < n (n <= 64): the positions of a multi-position prefill group.
void launch_set_positions(int* pos, int n, int p0, hipStream_t s);
// p[r] = v for r < n (n <= 64).
void launch_fill_i32(int* p, int n, int v, hipStream_t s);
// Opens request r of a slotted batch: position 0, live, its parameters and conditioning length.
void launch_slot_open(int* pos, int* live, ReqParams* par, int* nc, int r, const ReqParams& p, int n_ctx,
                      hipStream_t s);
// fills n launch-timing slots (STAMP_SUB sub-slots each) with {UINT64_MAX, 0}
// A x for an adapter (w = A as an f32 matrix [rank][in]; pro LN or F32 with x / x_stride /
// ln_*; y = [col][y_stride]), the column built as the adapted projection builds it
void launch_adapter_ax(const GemvArgs& a, hipStream_t s);
void launch_stamp_init(unsigned long long* p, int n, hipStream_t s);
// DoRA rows (lora.h:11-32, 142): norm[r] = sqrt(||W_r||^2 + 2s<W_r,(BA)_r> + s^2||(BA)_r||^2)
// from the dequantized base rows, in double; bad != 0 afterwards if a base weight was not finite
void launch_dora_norm(const DevMat& w, const float* A, const float* B, int rank, float scale, float* norm, int* bad,
                      hipStream_t s);
void launch_repack(int type, const uint8_t* raw, int64_t rows, int in, void* q, uint16_t* d, hipStream_t s);

// T5 encoder pieces (src/ac/t5.h:85-140):
// rows of a matrix (ggml get_rows): out[t][i] = m row ids[t], element i, for n ids
void launch_rows(const DevMat& m, const int32_t* ids, int n, float* out, hipStream_t s);
// RMS norm of ncol columns of n elements (stride apart): (x * (1 / sqrtf(mean(x^2) + eps))) * w
void launch_rms(const float* x, int n, int ncol, int stride, const float* w, float eps, float* y, hipStream_t s);
// bias[(h * seq + q) * seq + k] = table row rel[k - q + zero], element h, + 0 (rel: the bucket
// of each relative position key - query, position 0 at index zero)
void launch_t5_bias(const DevMat& table, const int32_t* rel, int zero, int seq, int heads, float* bias, hipStream_t s);
// ReLU of ncol columns of n f32 values into the activation form of the consumer's weights
void launch_relu_act(const float* x, int n, int ncol, const ActBuf& dst, hipStream_t s);

}  // namespace mgx
