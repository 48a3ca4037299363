/*
 * mgx.h -- C ABI of the MI355X (gfx950) MusicGen LM decode library.
 *
 * It replaces the ggml graph behind audiocraft.cpp's `ac::mg_generate` (src/mg/pipeline.cpp:
 * 199-314): the `Decoder` class (pipeline.cpp:36-195) becomes an `mgx_stream`, the weights the
 * `GgufModel` holds (src/gguf_model.h:241-346) become an `mgx_model`, and the loop body --
 * forward, classifier-free-guidance mix and top-k sampling -- runs on the GPU. GGUF parsing, T5,
 * the delay pattern's host bookkeeping, EnCodec and HTTP stay with the caller.
 *
 * Conventions: plain pointers and sizes; the caller owns every host buffer it passes; all
 * host pointers are read or written before the call returns. Every entry point returns
 * MGX_OK (0) or a negative status, with a message in mgx_last_error() (thread-local) -- the
 * reference throws std::runtime_error at the same sites (kv_cache.h:73-77, pipeline.cpp:81-83,
 * 98-99, 204-212; gguf_model.h:425-436), and a C++ caller rethrows the message.
 *
 * Threading: one caller thread per stream; distinct streams may be driven from distinct
 * threads. The reference's server runs one job at a time (src/serve/http.h:201-205); the
 * request server below (mgx_server_*) takes concurrent callers into one batched decode.
 */
#ifndef MGX_H
#define MGX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    MGX_OK = 0,
    MGX_ERR_INVALID = -1,   /* bad argument, shape or tensor */
    MGX_ERR_DEVICE = -2,    /* HIP runtime or allocation failure */
    MGX_ERR_OVERFLOW = -3,  /* KV cache overflow (kv_cache.h:73-77) */
    MGX_ERR_STATE = -4      /* multi-token forward after history (pipeline.cpp:81-83) */
};

/* ggml type ids accepted for weight matrices (gguf_model.h passes them through). */
enum { MGX_TYPE_F32 = 0, MGX_TYPE_F16 = 1, MGX_TYPE_Q4_0 = 2, MGX_TYPE_Q8_0 = 8 };

typedef struct mgx_model mgx_model;
typedef struct mgx_stream mgx_stream;

/* ac::LmConfig (src/mg/lm.h:42-93), the `ac.lm.*` GGUF metadata. */
typedef struct mgx_lm_config {
    int32_t dim, layers, heads, head_dim, ff_dim, cond_dim, n_q, card, special_token_id, pos_denominator;
    float max_period, norm_eps, cfg_coef;
} mgx_lm_config;

/* One GGUF tensor as ggml holds it: name (tools/convert_musicgen_lm.py:149-210), ggml type,
   ne[] in ggml order (ne[0] contiguous), and the raw tensor bytes (ggml block layout). */
typedef struct mgx_tensor {
    const char* name;
    int32_t type;
    int64_t ne[4];
    const void* data;
    uint64_t nbytes;
} mgx_tensor;

/* One adapted projection, ac::LoraProjection (src/ac/lora.h:39-47) as load_lora builds it
   (lora.h:113-176): A ggml [in, rank], B ggml [rank, out], f32; magnitude [out] for
   "dora-rows" adapters, NULL for "lora". */
typedef struct mgx_adapter {
    const char* target;      /* "lm.<i>.{self.qkv,self.out,cross.q,cross.kv,cross.out,ff.0,ff.2}.weight" */
    const float* A;
    const float* B;
    const float* magnitude;
    int32_t rank;
    float alpha;
    float strength;
} mgx_adapter;

/* Replaces load_gguf's device upload (gguf_model.h:363-414) and LmConfig::from's checks
   (lm.h:60-90): validates names, shapes and types and uploads the weights to the current
   HIP device once. `tensors` may be freed after the call. */
int mgx_model_create(const mgx_lm_config* cfg, const mgx_tensor* tensors, int32_t n_tensors, mgx_model** out);

/* Attaches adapters (load_mg_lora, lora.h:195-210) for every stream and session created
   afterwards; the reference passes its LoraMap to mg_generate (pipeline.h:63-67). Checks as
   load_lora does (lora.h:113-176): a supported target, rank > 0, finite alpha > 0 and
   strength, finite A, B and magnitude; in addition rank <= 64 and one adapter per target.
   DoRA rows on a quantized base use the dequantized base rows for ||W||^2 (the reference
   throws there, lora.h:11-13). n == 0 detaches. MGX_ERR_STATE while any stream or session of
   the model exists. The host arrays may be freed after the call. */
int mgx_model_set_adapters(mgx_model* model, const mgx_adapter* adapters, int32_t n);

void mgx_model_destroy(mgx_model* model);

/* Decoder's constructor (pipeline.cpp:38-47): a KV cache of `capacity` positions for `n_seq`
   streams (2 = guided: stream 0 conditional, stream 1 null). With `cross_attention` set,
   `t5_hidden` [n_ctx][cond_dim] f32 is projected through lm.cond_proj once into stream 0
   (stream 1 stays zero, pipeline.cpp:135-180) and every layer's cross.kv is projected from it
   once as well (the reference recomputes it each step, lm.h:184; the values are the same). */
int mgx_stream_create(mgx_model* model, int32_t capacity, int32_t n_seq, const float* t5_hidden, int32_t n_ctx,
                      int32_t cross_attention, mgx_stream** out);

/* Decoder::forward (pipeline.cpp:59-132): feeds n_tokens sequence steps, ids [n_q][n_tokens]
   codebook-major, and writes the last step's logits [n_seq][n_q][card] (ggml [card, n_q,
   n_seq]). A multi-token call is a prefill and needs an empty cache. */
int mgx_forward(mgx_stream* stream, const int32_t* ids, int32_t n_tokens, float* logits_out);

/* KvCache::reset / used / Decoder::forwards / cache_bytes (kv_cache.h:69-81, pipeline.cpp:54-55). */
int mgx_stream_reset(mgx_stream* stream);
int32_t mgx_stream_used(const mgx_stream* stream);
int32_t mgx_stream_forwards(const mgx_stream* stream);
uint64_t mgx_stream_cache_bytes(const mgx_stream* stream);
void mgx_stream_destroy(mgx_stream* stream);

/* mg_use_guidance (pipeline.h:41-43). */
int32_t mgx_use_guidance(float cfg_coef, int32_t description_empty);

/* GenerateParams (pipeline.h:25-34). */
typedef struct mgx_generate_params {
    int32_t max_gen_len;
    int32_t use_sampling;
    float temperature;
    int32_t top_k;
    float cfg_coef;
    uint64_t seed;
} mgx_generate_params;

/* GenerateReport (pipeline.h:45-56); first_logits is returned through its own buffer. */
typedef struct mgx_generate_report {
    uint64_t cache_bytes;
    int32_t prefill_tokens;
    int32_t decode_steps;
    int32_t forwards;
    double prefill_seconds;
    double decode_seconds;
} mgx_generate_report;

/* ac::mg_generate (pipeline.cpp:199-314): prompt_codes [n_q][prompt_len], t5_hidden
   [n_ctx][cond_dim]; codes_out [n_q][max_gen_len] (prompt included); first_logits_out
   [n_q][card] (the guided mix of the first prediction, pipeline.cpp:275-276);
   step_logits_out, if not NULL, [S - start][n_q][card] with the mixed logits of every
   forward. The sampling stream is the reference's: mt19937(seed), one uniform per sampled
   (step, codebook) slot in step-then-codebook order (pipeline.cpp:278-288, rng.h:20-22). */
int mgx_generate(mgx_model* model, const float* t5_hidden, int32_t n_ctx, int32_t description_empty,
                 const int32_t* prompt_codes, int32_t prompt_len, const mgx_generate_params* params,
                 int32_t* codes_out, float* first_logits_out, float* step_logits_out,
                 mgx_generate_report* report);

/* mg_generate in resumable pieces, for callers that report progress after every step as
   the reference's ProgressFn does (pipeline.cpp:301) or time a subset of the steps.
   mgx_session_create builds the delay-pattern sequence, the pre-drawn uniform stream and a
   stream, and runs nothing. mgx_session_step runs up to n_forwards more loop iterations --
   the first is the prefill of the prompt, the rest single-token decodes -- each ending with
   the on-device CFG mix, sampling and sequence write, then waits for them; *done gets the
   count. mgx_session_finish reads the codes back (reverted, pipeline.cpp:307-313; the
   final check only once every step has run), the first logits, the per-step logits when
   keep_step_logits was set, and the report. */
typedef struct mgx_session mgx_session;
int mgx_session_create(mgx_model* model, const float* t5_hidden, int32_t n_ctx, int32_t description_empty,
                       const int32_t* prompt_codes, int32_t prompt_len, const mgx_generate_params* params,
                       int32_t keep_step_logits, mgx_session** out);
int mgx_session_step(mgx_session* session, int32_t n_forwards, int32_t* done);
int32_t mgx_session_remaining(const mgx_session* session);
int mgx_session_finish(mgx_session* session, int32_t* codes_out, float* first_logits_out, float* step_logits_out,
                       mgx_generate_report* report);
void mgx_session_destroy(mgx_session* session);

/* Batched decode of several requests in lockstep (no reference counterpart: the reference
   runs one job at a time, src/serve/http.h:201-205; each request is mg_generate,
   pipeline.cpp:199-314). The requests share the prompt length, max_gen_len, the conditioning
   length n_ctx and whether guidance is on (mg_use_guidance); each has its own conditioning,
   prompt, seed, sampling parameters and cfg_coef, and its own KV cache. At most 16 streams:
   16 unguided or 8 guided requests. Every request's codes, first logits and per-step logits
   equal those of mgx_generate on that request alone. Step, profile and destroy through the
   mgx_session_* calls; mgx_session_finish reads request 0. */
typedef struct mgx_batch_request {
    const float* t5_hidden;          /* [n_ctx][cond_dim] */
    int32_t description_empty;
    const int32_t* prompt_codes;     /* [n_q][prompt_len] */
    mgx_generate_params params;
} mgx_batch_request;
int mgx_batch_create(mgx_model* model, const mgx_batch_request* requests, int32_t n_requests, int32_t n_ctx,
                     int32_t prompt_len, int32_t keep_step_logits, mgx_session** out);
int mgx_batch_finish(mgx_session* session, int32_t request, int32_t* codes_out, float* first_logits_out,
                     float* step_logits_out, mgx_generate_report* report);
int32_t mgx_session_requests(const mgx_session* session);

/* A request server: many concurrent callers, one batched decode on the GPU. It replaces the
   reference services' one-job-at-a-time generation lock (Sessions::gpu() held for the whole
   of mg_generate, src/serve/http.h:201-205, 254-255, 278-291; the job start of
   tools/musicgen-server.cpp:321-390): each job thread calls mgx_server_generate where it
   called mg_generate, and blocks until its result is ready. One worker thread owns `slots`
   request slots; between rounds of at most steps_per_round batch steps it admits queued
   requests into free slots (first come, first served). A request's prompt is prefilled into
   its slot at admission (256 positions per step when guided), then its loop runs in the batch steps; its
   slot frees after its own last step. Requests in
   one batch differ in anything: prompt and generation length (up to max_gen_len),
   conditioning (up to max_ctx tokens), guidance, seed and sampling parameters; each one's
   codes, first logits and per-step logits equal mgx_generate's for it alone.
   guided = 1: slots of two streams (guided and unguided requests); 0: one stream per slot
   (unguided requests only, up to 16 slots). keep_step_logits: mgx_server_generate may ask for
   per-step logits. steps_per_round 0 means 16.
   progress, if not NULL, gets (user, done, total) after every loop iteration as the
   reference's ProgressFn (pipeline.cpp:301), called from the worker thread after the round
   that ran it. Errors: argument checks fail at once with mg_generate's messages; a device
   error fails every request in the server and every later call; mgx_server_destroy fails the
   requests still waiting (MGX_ERR_STATE) and returns once their callers have returned. */
typedef struct mgx_server mgx_server;
typedef struct mgx_server_config {
    int32_t slots;
    int32_t guided;
    int32_t max_gen_len;
    int32_t max_ctx;
    int32_t keep_step_logits;
    int32_t steps_per_round;
} mgx_server_config;
typedef void (*mgx_progress_fn)(void* user, int32_t done, int32_t total);
typedef struct mgx_server_counters {
    int64_t steps;        /* batch steps run */
    int64_t slot_steps;   /* sum over steps of the requests they advanced */
    int64_t served;       /* requests completed */
    int32_t active;       /* requests in slots */
    int32_t queued;       /* requests waiting for a slot */
} mgx_server_counters;
int mgx_server_create(mgx_model* model, const mgx_server_config* config, mgx_server** out);
int mgx_server_generate(mgx_server* server, const float* t5_hidden, int32_t n_ctx, int32_t description_empty,
                        const int32_t* prompt_codes, int32_t prompt_len, const mgx_generate_params* params,
                        mgx_progress_fn progress, void* user, int32_t* codes_out, float* first_logits_out,
                        float* step_logits_out, mgx_generate_report* report);
int mgx_server_stats(mgx_server* server, mgx_server_counters* out);
void mgx_server_destroy(mgx_server* server);

/* Launch timing (no reference counterpart; the reference has wall clocks only,
   pipeline.cpp:15-18): with every > 0, every `every`-th loop iteration runs outside the
   captured graph (same kernels, launched one by one) and each of its GEMV (kind 0) and
   self-attention (kind 1) and cross-attention (kind 9) launches records its span on the GPU's
   constant-rate wall clock
   (earliest block start to latest wave end -- a kernel tracer's duration; for attention, the
   chunk kernel's first block start to the combine kernel's last wave end, the boundary between
   them included). profile_read sums those milliseconds, the algorithmic bytes (weights at their stored
   precision; f32 K and V of the keys attended) and the launch count, for one kind of launch:
   MGX_PROF_GEMV every weight GEMV, MGX_PROF_ATTN the self-attention, MGX_PROF_XATTN the
   cross-attention, or the GEMV of one projection (its adapter's A x launch, if any, is not
   included). */
enum {
    MGX_PROF_GEMV = 0, MGX_PROF_ATTN = 1, MGX_PROF_QKV = 2, MGX_PROF_OUT = 3, MGX_PROF_CROSS_Q = 4,
    MGX_PROF_CROSS_OUT = 5, MGX_PROF_FF0 = 6, MGX_PROF_FF2 = 7, MGX_PROF_HEADS = 8, MGX_PROF_XATTN = 9
};
int mgx_session_profile(mgx_session* session, int32_t every);
int mgx_session_profile_read(mgx_session* session, int32_t kind, double* ms_total, double* bytes_total,
                             int32_t* launches);
/* The hipStream_t the session's kernels run on. */
void* mgx_session_hip_stream(mgx_session* session);

/* GGUF files without ggml: GgufModel / load_gguf (src/gguf_model.h:241-414) for what the LM
   needs. mgx_gguf_open maps the file read-only and checks the header, every key/value and every
   tensor's extent against the file size (load_gguf's short-read check, gguf_model.h:384-389);
   GGUF v2 and v3, tensor types F32 / F16 / BF16 / Q4_0 / Q4_1 / Q5_0 / Q5_1 / Q8_0. Tensor data
   pointers point into the mapping and stay valid until mgx_gguf_close. */
typedef struct mgx_gguf mgx_gguf;
int mgx_gguf_open(const char* path, mgx_gguf** out);
void mgx_gguf_close(mgx_gguf* gguf);
int32_t mgx_gguf_tensor_count(const mgx_gguf* gguf);
int mgx_gguf_tensor(const mgx_gguf* gguf, int32_t index, mgx_tensor* out);
int mgx_gguf_find_tensor(const mgx_gguf* gguf, const char* name, mgx_tensor* out);   /* GgufModel::get */
/* GgufModel::u32 / f32 / string (gguf_model.h:273-305): "missing key: ..." or a type error. */
int mgx_gguf_u32(const mgx_gguf* gguf, const char* key, uint32_t* out);
int mgx_gguf_f32(const mgx_gguf* gguf, const char* key, float* out);
int mgx_gguf_string(const mgx_gguf* gguf, const char* key, char* buf, uint64_t capacity, uint64_t* length);
/* LmConfig::from (src/mg/lm.h:60-90): the ac.* keys and their checks. */
int mgx_gguf_lm_config(const mgx_gguf* gguf, mgx_lm_config* out);
/* load_gguf + LmConfig::from + mgx_model_create in one call; the file may be closed afterwards. */
int mgx_model_create_from_gguf(const mgx_gguf* gguf, mgx_model** out);
/* load_mg_lora (lora.h:113-176, 195-210) on an adapter file (general.architecture
   "ac-musicgen-lora"): version, rank, alpha, type, the .lora_A / .lora_B (/ .magnitude) tensors
   and their shapes against the model, the base-name check when `base` is given; then
   mgx_model_set_adapters. The adapter file must stay open while the call runs only. */
int mgx_model_set_adapters_from_gguf(mgx_model* model, const mgx_gguf* adapter, const mgx_gguf* base, float strength);

/* The message of the last failed call on this thread. */
const char* mgx_last_error(void);

/* The T5-base text encoder (ac::T5EncoderConfig / ac::t5_encode, src/ac/t5.h:20-140, as
   ac::encode_prompt runs it, src/ac/conditioner.h:56-108: one prompt at its own token count,
   no padding). The reference loads the encoder from its GGUF and frees it in every call; an
   mgx_t5 stays resident on the current HIP device and mgx_t5_encode is only the forward:
   ids [n_tokens] (the tokenizer's output, 1 to 256 tokens) -> hidden_out [n_tokens][dim], the
   last hidden state TextCondition::hidden holds. Tensors as tools/convert_t5.py:107-119 names
   them: te.embed.weight, te.relative_attention_bias.weight (F32 or F16), te.<i>.{attn_norm,
   q,k,v,o,ffn_norm,wi,wo}.weight, te.norm.weight; matrices F32 / F16 / Q8_0 / Q4_0, norms F32.
   head_dim must be 64. One encode at a time per encoder (calls from several threads wait for
   each other). */
typedef struct mgx_t5_config {
    int32_t dim, layers, heads, head_dim, intermediate, vocab, relative_buckets, relative_max_distance;
    float eps;
} mgx_t5_config;
typedef struct mgx_t5 mgx_t5;
int mgx_t5_create(const mgx_t5_config* config, const mgx_tensor* tensors, int32_t n_tensors, mgx_t5** out);
/* T5EncoderConfig::from (t5.h:31-43) and the encoder straight from its GGUF file. */
int mgx_gguf_t5_config(const mgx_gguf* file, mgx_t5_config* out);
int mgx_t5_create_from_gguf(const mgx_gguf* file, mgx_t5** out);
int mgx_t5_encode(mgx_t5* t5, const int32_t* ids, int32_t n_tokens, float* hidden_out);
/* mgx_t5_encode without any allocation: every working buffer of the encode (ids, relative
   buckets, hidden states, q / k / v, attention bias, activation forms) lives in one file-scope
   device array of 32 MiB that each device running the call holds until the process ends. No
   counterpart in the reference: it is for callers that cannot allocate device memory while
   they run (tight serving loops, code around HIP graph capture). Same arguments and results as
   mgx_t5_encode (bit for bit); MGX_ERR_INVALID when the encode needs more than 32 MiB
   (about n_tokens * (2 dim + 6 heads*64 + 2 intermediate) * 4 + heads * n_tokens^2 * 4 bytes:
   15 MiB for T5-base at 256 tokens). Calls share the array: calls that overlap on one device
   race (the encoder's own lock serializes calls on one mgx_t5). */
int mgx_t5_encode_static(mgx_t5* t5, const int32_t* ids, int32_t n_tokens, float* hidden_out);
void mgx_t5_destroy(mgx_t5* t5);
/* t5_relative_position_bucket (t5.h:46-61): relative_position = key - query. */
int32_t mgx_t5_relative_bucket(int32_t relative_position, int32_t num_buckets, int32_t max_distance);

/* The EnCodec decoder: RVQ codes -> audio (rvq_decode, src/mg/encodec.h:69-84; codec_decode,
   src/ac/codec.h:127-146, over seanet_decode_pre / lstm_graph / seanet_decode_post,
   src/ac/seanet.h:282-317, src/ac/lstm.h:44-101), resident on the current HIP device. The
   config is SeanetConfig (seanet.h:32-92); only ELU codecs (MusicGen's EnCodec) are accepted.
   Tensors as tools/convert_seanet.py names them, all f32: codec.decoder.in.{weight,bias},
   codec.decoder.lstm.<l>.{w_ih,w_hh,bias}, codec.decoder.stage.<s>.up.{weight_col2im,bias},
   codec.decoder.stage.<s>.res.<j>.conv{1,2}.{weight,bias}, codec.decoder.out.{weight,bias},
   codec.rvq.<i>.embed. codes [rvq_n_q][frames] -> audio_out [channels][frames * hop_length];
   mgx_codec_decode_latent takes the latent [latent_dim][frames] instead. f32 throughout; the
   result equals the reference's within f32 rounding. One decode at a time per codec. */
typedef struct mgx_codec_config {
    int32_t channels, n_filters, n_residual_layers, kernel_size, residual_kernel_size, last_kernel_size;
    int32_t dilation_base, compress, lstm_layers, latent_dim, sample_rate, hop_length, frame_rate;
    int32_t rvq, rvq_n_q, rvq_bins;   /* rvq: 1 when the quantizer is "rvq" */
    int32_t elu;                      /* 1 when the activation is "ELU" */
    int32_t n_ratios;
    int32_t ratios[8];                /* decoder order */
} mgx_codec_config;
typedef struct mgx_codec mgx_codec;
int mgx_codec_create(const mgx_codec_config* config, const mgx_tensor* tensors, int32_t n_tensors, mgx_codec** out);
/* SeanetConfig::from (seanet.h:60-92) and the decoder straight from the codec's GGUF file. */
int mgx_gguf_codec_config(const mgx_gguf* file, mgx_codec_config* out);
int mgx_codec_create_from_gguf(const mgx_gguf* file, mgx_codec** out);
int mgx_codec_decode(mgx_codec* codec, const int32_t* codes, int32_t frames, float* audio_out);
int mgx_codec_decode_latent(mgx_codec* codec, const float* latent, int32_t frames, float* audio_out);
void mgx_codec_destroy(mgx_codec* codec);

#ifdef __cplusplus
}
#endif

#endif /* MGX_H */
