/*
 * oracle/cpu_ref.c -- CPU restatement of audiocraft.cpp's MusicGen LM decode path.
 *
 * TEST INFRASTRUCTURE, NOT PRODUCT CODE. This library is the parity oracle for the HIP
 * library and the timed CPU baseline ("port"). Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg load it, and only as the checker. The product path never
 * links, loads or calls anything here.
 *
 * What it restates (file:line in the reference, audiocraft.cpp v0.1.4):
 *   sin_positions ............ src/mg/lm.h:102-116
 *   layer_norm ............... src/ac/transformer.h:28-38 (ggml_norm -> mul -> add)
 *   lora_linear / mul_mat .... src/ac/lora.h:50-83 (plain and DoRA-rows)
 *   lm_layer ................. src/mg/lm.h:152-204
 *   lm_forward ............... src/mg/lm.h:225-259
 *   lm_project_context ....... src/mg/lm.h:265-269, src/mg/pipeline.cpp:144-180
 *   KvCache .................. src/mg/kv_cache.h:33-115 (f32, K [hd,cap,H,N], V^T [cap,hd,H,N])
 *   nn::sdpa_vt .............. src/nn.h:186-191
 *   Decoder::forward ......... src/mg/pipeline.cpp:59-132
 *   mg_generate .............. src/mg/pipeline.cpp:199-314
 *   mg_use_guidance .......... src/mg/pipeline.h:41-43
 *   sampling ................. src/mg/sampling.h:32-105
 *   Rng ...................... src/rng.h:15-33
 *   DelayPattern ............. src/mg/pattern.h:31-115
 *   t5_encode / buckets ...... src/ac/t5.h:46-140 (T5-base encoder, conditioner.h:56-108)
 *
 * The reference does every tensor op through ggml (submodule betweentwomidnights/ggml @
 * e3db5210), which is not vendored, so the ggml CPU kernels' bit-level behaviour cannot be
 * pinned. This file fixes one convention for each of them and keeps it; every choice below
 * is a legal ggml-CPU behaviour (ggml's own SIMD variants differ from each other in the
 * same places):
 *
 *   mul_mat, quantized weights (Q8_0, Q4_0): the activation column is quantized to Q8_0
 *     per 32-block (d = amax/127, id = d ? 1/d : 0, q = roundf(x*id), d stored fp16 RNE);
 *     each block gives an exact integer dot `isum`; its term is (float)isum * (dw*dx) with
 *     dw, dx the fp16 scales widened to f32 (their product is exact); the terms of one row
 *     are summed in f32 as 64 strided partials (block b -> partial b mod 64, each partial
 *     accumulated in increasing b) folded by a butterfly (off = 32,16,..,1:
 *     p[l] = p[l] + p[l+off]).
 *   mul_mat, F16 weights: the activation is rounded to fp16 (RNE); products are exact in
 *     f32; 8-element chunks, chunk c -> partial c mod 64, fmaf in increasing element
 *     order inside a partial, same butterfly. F32 weights: same, without the rounding.
 *   norm: mean and variance as double sums, element i -> partial (i/4) mod 256 accumulated
 *     in increasing i, folded by a 256-wide butterfly (off = 128,..,1); result (x - mean) *
 *     (1.0f / sqrtf(var + eps)), then * w, then + b, each rounded in f32.
 *   soft_max_ext + the V^T mul_mat, per 64-key chunk: x*scale (+mask); the chunk's max;
 *     e = expf(x - chunk max); the chunk's sum of e in double (64-wide butterfly); V^T.e as
 *     16 partials (key j -> partial j mod 16, fmaf in increasing j) + butterfly. The chunks
 *     are then combined with their weights exp(chunk max - max) in double: the total is the
 *     64-wide butterfly of the chunks' (sum * weight), and each chunk's V^T.e enters the
 *     output, in chunk order, through an fmaf by (float)(weight / total). q.k: 16 partials
 *     (dim i -> partial (i/4) mod 16, fmaf in order) + butterfly.
 *   gelu_erf: 0.5f*x*(1.0f+erff(x*0.70710678f)).
 *   expf / erff: (float) of this file's own double exp (Cody-Waite reduction by ln2 split
 *     hi/lo, degree-13 Taylor, ldexp) and double erf (two Chebyshev interpolants, below
 *     |x| = 1 and on [1, 4), +-1 beyond; absolute error under 1.3e-12). The f32 results are
 *     within one ulp of the true functions (the correctly rounded value but for ~1e-8 of
 *     expf and ~1e-4 of erff arguments).
 *
 * Every floating-point step is written out (the file is compiled with -ffp-contract=off),
 * so the HIP kernels can reproduce it bit for bit.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#ifdef _OPENMP
#include <omp.h>
#endif
#ifdef __AVX2__
#include <immintrin.h>
#endif

#define REF_API __attribute__((visibility("default")))

enum { T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q8_0 = 8 };

static __thread char g_err[512];
static void set_err(const char* msg) { snprintf(g_err, sizeof g_err, "%s", msg); }
REF_API const char* ref_last_error(void) { return g_err; }

/* ------------------------------------------------------------------------------------ */
/* fp16                                                                                 */
/* ------------------------------------------------------------------------------------ */
REF_API float ref_fp16_to_fp32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu, man = h & 0x3ffu, bits;
    if (exp == 0) {
        if (man == 0) bits = sign;
        else {                                   /* subnormal: renormalize */
            int e = -1;
            do { ++e; man <<= 1; } while (!(man & 0x400u));
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3ffu) << 13);
        }
    } else if (exp == 31) bits = sign | 0x7f800000u | (man << 13);
    else bits = sign | ((exp + 112u) << 23) | (man << 13);
    float f; memcpy(&f, &bits, 4); return f;
}

/* Round-to-nearest-even f32 -> fp16 (what _cvtss_sh(x, 0) and the scalar table do). */
REF_API uint16_t ref_fp32_to_fp16(float f) {
    uint32_t x; memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);          /* rounds to inf */
    if (ax < 0x38800000u) {                                             /* fp16 subnormal */
        if (ax < 0x33000000u) return (uint16_t)sign;                    /* < half min sub */
        const int e = (int)(ax >> 23);
        const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        const int shift = 126 - e;                                      /* 14..24 */
        uint32_t r = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (r & 1u))) ++r;
        return (uint16_t)(sign | r);
    }
    uint32_t r = ((ax >> 13) - (112u << 10));
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) ++r;
    return (uint16_t)(sign | r);
}

static inline float f16at(const uint8_t* p) {
    uint16_t h; memcpy(&h, p, 2);
#ifdef __F16C__
    return _cvtsh_ss(h);                         /* exact widening, same as the table */
#else
    return ref_fp16_to_fp32(h);
#endif
}

/* ------------------------------------------------------------------------------------ */
/* exp / erf                                                                            */
/* ------------------------------------------------------------------------------------ */
static const double RECIP_FACT[14] = {
    1.0, 1.0, 0.5, 0.16666666666666666, 0.041666666666666664, 0.008333333333333333,
    0.001388888888888889, 0.0001984126984126984, 2.48015873015873e-05,
    2.7557319223985893e-06, 2.755731922398589e-07, 2.505210838544172e-08,
    2.08767569878681e-09, 1.6059043836821613e-10};

REF_API double ref_exp(double x) {
    if (x != x) return x;
    if (x > 709.782712893384) return INFINITY;
    if (x < -745.2) return 0.0;
    const double k = rint(x * 1.4426950408889634);
    double r = fma(-k, 0.6931471805599453, x);
    r = fma(-k, 2.3190468138462996e-17, r);
    double p = RECIP_FACT[13];
    for (int n = 12; n >= 0; --n) p = fma(p, r, RECIP_FACT[n]);
    return ldexp(p, (int)k);
}
REF_API float ref_expf(float x) { return (float)ref_exp((double)x); }

/* erf: two Chebyshev interpolants in monomial form (audiocraft.cpp_amd/csrc/erf_coeffs.py derives
   them from 40-digit erf values): |x| < 1: x * P(2x^2 - 1), P of degree 11; 1 <= |x| < 4:
   1 - Q(t), t = |x| * 2/3 - 5/3, Q (erfc on [1, 4]) of degree 20; +-1 beyond. Absolute error
   below 1.5e-15 and 1.3e-12 (measured against mpmath). The GPU kernels evaluate the same
   steps with the same constants. */
static const double ERF_P[12] = {
    0x1.ee51eb23cb7ebp-1, -0x1.1fd162921520ep-3, 0x1.454368017b319p-6,
    -0x1.2b902b7b26e28p-9, 0x1.c82aa24968f47p-13, -0x1.263991d3aca15p-16,
    0x1.4866394fa4c3ep-20, -0x1.429e4c163b13bp-24, 0x1.1ad503d95b599p-28,
    -0x1.c02cc0da54c52p-33, 0x1.4424c09b26e7bp-37, -0x1.2d4c29f5686cbp-42};
static const double ERF_Q[21] = {
    0x1.aab859b20b140p-12, -0x1.ac44a2cdb3c80p-9, 0x1.9180586b55ae8p-7,
    -0x1.cdb9fd59ee319p-6, 0x1.65964ef5668ffp-5, -0x1.7c8c5ebf7f0ccp-5,
    0x1.0521f53919ddep-5, -0x1.2faaceec90308p-7, -0x1.b5d2183e391e9p-8,
    0x1.3b371adacbf70p-7, -0x1.29d400459d61ep-8, -0x1.ca1cf08ac8d5dp-12,
    0x1.df3c4bd10ee4ep-10, -0x1.e7099cc2c7d56p-11, -0x1.d14ddd0a26b51p-15,
    0x1.3dc0c2909a110p-12, -0x1.e193532b72642p-14, -0x1.3af7b90db0f1ap-15,
    0x1.17a5709f8fe8ap-15, 0x1.048f70bb1e4f4p-20, -0x1.e180cb94805c1p-19};

REF_API double ref_erf(double x) {
    const double ax = fabs(x);
    if (ax < 1.0) {
        const double t = fma(2.0 * x, x, -1.0);
        double p = ERF_P[11];
        for (int n = 10; n >= 0; --n) p = fma(p, t, ERF_P[n]);
        return x * p;
    }
    if (ax >= 4.0) return x > 0 ? 1.0 : -1.0;
    const double t = fma(ax, 0x1.5555555555555p-1, -0x1.aaaaaaaaaaaabp+0);
    double p = ERF_Q[20];
    for (int n = 19; n >= 0; --n) p = fma(p, t, ERF_Q[n]);
    const double r = 1.0 - p;
    return x > 0 ? r : -r;
}
REF_API float ref_erff(float x) { return (float)ref_erf((double)x); }

/* ggml_gelu_erf (lm.h:203): 0.5*x*(1+erf(x/sqrt 2)) in f32. */
REF_API float ref_gelu_erf(float x) {
    const float e = ref_erff(x * 0.70710678118654752440f);
    return 0.5f * x * (1.0f + e);
}

/* ------------------------------------------------------------------------------------ */
/* ordered sums                                                                         */
/* ------------------------------------------------------------------------------------ */
static inline float fold_f(float* p, int w) {
    for (int off = w >> 1; off >= 1; off >>= 1)
        for (int l = 0; l < off; ++l) p[l] = p[l] + p[l + off];
    return p[0];
}
static inline double fold_d(double* p, int w) {
    for (int off = w >> 1; off >= 1; off >>= 1)
        for (int l = 0; l < off; ++l) p[l] = p[l] + p[l + off];
    return p[0];
}

/* ------------------------------------------------------------------------------------ */
/* quantization (ggml block layouts)                                                    */
/* ------------------------------------------------------------------------------------ */
/* Activation quantization to Q8_0 (ggml quantize_row_q8_0, scalar form). qs: int8 [n],
   d: the stored fp16 scale widened back to f32, one per 32-block. */
static void quantize_q8_act(const float* x, int n, int8_t* qs, float* d) {
    for (int b = 0; b < n / 32; ++b) {
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) {
            const float a = fabsf(x[b * 32 + j]);
            amax = amax > a ? amax : a;
        }
        const float dd = amax / 127.0f;
        const float id = dd != 0.0f ? 1.0f / dd : 0.0f;
        d[b] = ref_fp16_to_fp32(ref_fp32_to_fp16(dd));
        for (int j = 0; j < 32; ++j) qs[b * 32 + j] = (int8_t)roundf(x[b * 32 + j] * id);
    }
}

/* Exposed so tests can hold the activation quantizer to ggml's block format. out: n/32
   blocks of {fp16 d; int8 q[32]}. */
REF_API void ref_quantize_q8_0(const float* x, int n, uint8_t* out) {
    int8_t qs[32]; float d;
    for (int b = 0; b < n / 32; ++b) {
        quantize_q8_act(x + b * 32, 32, qs, &d);
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) { const float a = fabsf(x[b * 32 + j]); amax = amax > a ? amax : a; }
        const uint16_t h = ref_fp32_to_fp16(amax / 127.0f);
        memcpy(out + b * 34, &h, 2);
        memcpy(out + b * 34 + 2, qs, 32);
    }
}

/* ------------------------------------------------------------------------------------ */
/* matrices                                                                             */
/* ------------------------------------------------------------------------------------ */
typedef struct {
    int type, in, out;
    size_t row_bytes;
    const uint8_t* data;
} mat_t;

static size_t row_bytes_of(int type, int in) {
    switch (type) {
    case T_F32: return (size_t)in * 4;
    case T_F16: return (size_t)in * 2;
    case T_Q8_0: return (size_t)(in / 32) * 34;
    case T_Q4_0: return (size_t)(in / 32) * 18;
    }
    return 0;
}

/* The activation column in the weight's vec_dot_type. */
typedef struct {
    int8_t* qs;  /* Q8_0 quants [in] */
    float* d;    /* Q8_0 scales [in/32] */
    float* f;    /* f32 (or fp16-valued f32) [in] */
} act_t;

#ifdef __AVX2__
/* In-register 8x8 transpose: r[k] lane e <- old r[e] lane k. */
static inline void transpose8(__m256* r) {
    const __m256 t0 = _mm256_unpacklo_ps(r[0], r[1]), t1 = _mm256_unpackhi_ps(r[0], r[1]);
    const __m256 t2 = _mm256_unpacklo_ps(r[2], r[3]), t3 = _mm256_unpackhi_ps(r[2], r[3]);
    const __m256 t4 = _mm256_unpacklo_ps(r[4], r[5]), t5 = _mm256_unpackhi_ps(r[4], r[5]);
    const __m256 t6 = _mm256_unpacklo_ps(r[6], r[7]), t7 = _mm256_unpackhi_ps(r[6], r[7]);
    const __m256 s0 = _mm256_shuffle_ps(t0, t2, 0x44), s1 = _mm256_shuffle_ps(t0, t2, 0xEE);
    const __m256 s2 = _mm256_shuffle_ps(t1, t3, 0x44), s3 = _mm256_shuffle_ps(t1, t3, 0xEE);
    const __m256 s4 = _mm256_shuffle_ps(t4, t6, 0x44), s5 = _mm256_shuffle_ps(t4, t6, 0xEE);
    const __m256 s6 = _mm256_shuffle_ps(t5, t7, 0x44), s7 = _mm256_shuffle_ps(t5, t7, 0xEE);
    r[0] = _mm256_permute2f128_ps(s0, s4, 0x20); r[1] = _mm256_permute2f128_ps(s1, s5, 0x20);
    r[2] = _mm256_permute2f128_ps(s2, s6, 0x20); r[3] = _mm256_permute2f128_ps(s3, s7, 0x20);
    r[4] = _mm256_permute2f128_ps(s0, s4, 0x31); r[5] = _mm256_permute2f128_ps(s1, s5, 0x31);
    r[6] = _mm256_permute2f128_ps(s2, s6, 0x31); r[7] = _mm256_permute2f128_ps(s3, s7, 0x31);
}
#endif

/* Exact integer dot of 32 int8 pairs (the order of integer adds does not matter). */
static inline int idot32(const int8_t* w, const int8_t* x) {
#ifdef __AVX2__
    const __m256i wv = _mm256_loadu_si256((const __m256i*)w), xv = _mm256_loadu_si256((const __m256i*)x);
    const __m256i p16 = _mm256_maddubs_epi16(_mm256_sign_epi8(wv, wv), _mm256_sign_epi8(xv, wv));
    const __m256i p32 = _mm256_madd_epi16(p16, _mm256_set1_epi16(1));
    __m128i s = _mm_add_epi32(_mm256_castsi256_si128(p32), _mm256_extracti128_si256(p32, 1));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0x4e));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0xb1));
    return _mm_cvtsi128_si32(s);
#else
    int isum = 0;
    for (int j = 0; j < 32; ++j) isum += (int)w[j] * (int)x[j];
    return isum;
#endif
}

static float dot_row(const mat_t* W, int r, const act_t* a, int c) {
    const uint8_t* row = W->data + (size_t)r * W->row_bytes;
    const int in = W->in;
    float part[64];
    for (int l = 0; l < 64; ++l) part[l] = 0.0f;
    if (W->type == T_Q8_0) {
        const int8_t* xq = a->qs + (size_t)c * in;
        const float* xd = a->d + (size_t)c * (in / 32);
        for (int b = 0; b < in / 32; ++b) {
            const uint8_t* blk = row + (size_t)b * 34;
            const int8_t* qw = (const int8_t*)(blk + 2);
            const int isum = idot32(qw, xq + b * 32);
            const float term = (float)isum * (f16at(blk) * xd[b]);
            part[b & 63] = part[b & 63] + term;
        }
    } else if (W->type == T_Q4_0) {
        const int8_t* xq = a->qs + (size_t)c * in;
        const float* xd = a->d + (size_t)c * (in / 32);
        for (int b = 0; b < in / 32; ++b) {
            const uint8_t* blk = row + (size_t)b * 18;
            const uint8_t* qs = blk + 2;
            int8_t wq[32];
            for (int j = 0; j < 16; ++j) { wq[j] = (int8_t)((qs[j] & 15) - 8); wq[j + 16] = (int8_t)((qs[j] >> 4) - 8); }
            const int isum = idot32(wq, xq + b * 32);
            const float term = (float)isum * (f16at(blk) * xd[b]);
            part[b & 63] = part[b & 63] + term;
        }
    } else {
        const float* x = a->f + (size_t)c * in;
#ifdef __AVX2__
        if (in % 64 == 0) {
            /* 8 consecutive chunks at a time: transpose so lane k of acc[g] is partial
               8g+k and the 8 fmaf of one chunk stay in element order. */
            __m256 acc[8];
            for (int g = 0; g < 8; ++g) acc[g] = _mm256_setzero_ps();
            for (int i0 = 0; i0 < in; i0 += 64) {
                __m256 w[8], xv[8];
                for (int k = 0; k < 8; ++k) {
                    if (W->type == T_F16) w[k] = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(row + (size_t)(i0 + 8 * k) * 2)));
                    else w[k] = _mm256_loadu_ps((const float*)row + i0 + 8 * k);
                    xv[k] = _mm256_loadu_ps(x + i0 + 8 * k);
                }
                transpose8(w); transpose8(xv);
                __m256 s = acc[(i0 >> 6) & 7];
                for (int e = 0; e < 8; ++e) s = _mm256_fmadd_ps(w[e], xv[e], s);
                acc[(i0 >> 6) & 7] = s;
            }
            for (int g = 0; g < 8; ++g) _mm256_storeu_ps(part + 8 * g, acc[g]);
            return fold_f(part, 64);
        }
#endif
        for (int i = 0; i < in; ++i) {
            const int l = (i >> 3) & 63;
            const float w = W->type == T_F16 ? f16at(row + (size_t)i * 2) : ((const float*)row)[i];
            part[l] = fmaf(w, x[i], part[l]);
        }
    }
    return fold_f(part, 64);
}

static void act_prepare(const mat_t* W, const float* X, int ncol, act_t* a) {
    const size_t n = (size_t)ncol * W->in;
    a->qs = NULL; a->d = NULL; a->f = NULL;
    if (W->type == T_Q8_0 || W->type == T_Q4_0) {
        a->qs = (int8_t*)malloc(n);
        a->d = (float*)malloc(n / 32 * sizeof(float));
        for (int c = 0; c < ncol; ++c)
            quantize_q8_act(X + (size_t)c * W->in, W->in, a->qs + (size_t)c * W->in,
                            a->d + (size_t)c * (W->in / 32));
    } else {
        a->f = (float*)malloc(n * sizeof(float));
        for (size_t i = 0; i < n; ++i)
            a->f[i] = W->type == T_F16 ? ref_fp16_to_fp32(ref_fp32_to_fp16(X[i])) : X[i];
    }
}
static void act_free(act_t* a) { free(a->qs); free(a->d); free(a->f); }

/* ------------------------------------------------------------------------------------ */
/* LoRA / DoRA-rows on a projection (lora.h:50-83)                                      */
/* ------------------------------------------------------------------------------------ */
typedef struct {
    const float* A;         /* [rank][in]  (ggml [in, rank]) */
    const float* B;         /* [out][rank] (ggml [rank, out]) */
    const float* magnitude; /* [out] or NULL for plain LoRA */
    float* base_norm_sq;    /* [out], DoRA only: computed at load (lora.h:11-32) */
    float* norm;            /* [out], DoRA only: sqrt(||W + sBA||^2), fixed per adapter */
    int rank;
    float scale, strength;
} adapter_t;

/* Y[c][out] = W X[c] (+ adapter) for ncol columns, restating lora_linear. */
static void matmul(const mat_t* W, const adapter_t* ad, const float* X, int ncol, float* Y) {
    act_t a;
    act_prepare(W, X, ncol, &a);
    #pragma omp parallel for schedule(static)
    for (int r = 0; r < W->out; ++r)
        for (int c = 0; c < ncol; ++c) Y[(size_t)c * W->out + r] = dot_row(W, r, &a, c);
    act_free(&a);
    if (!ad) return;
    if ((ad->magnitude && ad->strength == 0.0f) || (!ad->magnitude && ad->scale == 0.0f)) return;
    /* y = Wx + s * B(Ax): A and B are f32 matrices, so both products are f32 x f32
       mul_mats with the 8-chunk/64-partial order. */
    const int in = W->in, out = W->out, rk = ad->rank;
    float* ax = (float*)malloc(sizeof(float) * (size_t)ncol * rk);
    for (int c = 0; c < ncol; ++c)
        for (int k = 0; k < rk; ++k) {
            float part[64]; for (int l = 0; l < 64; ++l) part[l] = 0.0f;
            const float* x = X + (size_t)c * in;
            const float* arow = ad->A + (size_t)k * in;
            for (int i = 0; i < in; ++i) part[(i >> 3) & 63] = fmaf(arow[i], x[i], part[(i >> 3) & 63]);
            ax[(size_t)c * rk + k] = fold_f(part, 64);
        }
    #pragma omp parallel for schedule(static)
    for (int r = 0; r < out; ++r)
        for (int c = 0; c < ncol; ++c) {
            float part[64]; for (int l = 0; l < 64; ++l) part[l] = 0.0f;
            const float* brow = ad->B + (size_t)r * rk;
            for (int k = 0; k < rk; ++k) part[(k >> 3) & 63] = fmaf(brow[k], ax[(size_t)c * rk + k], part[(k >> 3) & 63]);
            const float lo = fold_f(part, 64) * ad->scale;     /* ggml_scale */
            float* y = &Y[(size_t)c * out + r];
            const float base = *y;
            float v = base + lo;                                 /* ggml_add */
            if (ad->magnitude) {
                v = v * (ad->magnitude[r] / ad->norm[r]);        /* ggml_mul(y, ggml_div(m, sqrt(nsq))) */
                if (ad->strength != 1.0f) v = base + (v - base) * ad->strength;
            }
            *y = v;
        }
    free(ax);
}

/* ------------------------------------------------------------------------------------ */
/* layer norm (transformer.h:28-38)                                                     */
/* ------------------------------------------------------------------------------------ */
REF_API void ref_layer_norm(const float* x, int n, const float* w, const float* b, float eps, float* y) {
    double part[256];
    for (int l = 0; l < 256; ++l) part[l] = 0.0;
    for (int i = 0; i < n; ++i) part[(i >> 2) & 255] = part[(i >> 2) & 255] + (double)x[i];
    const float mean = (float)(fold_d(part, 256) / (double)n);
    for (int l = 0; l < 256; ++l) part[l] = 0.0;
    for (int i = 0; i < n; ++i) {
        const float v = x[i] - mean;
        y[i] = v;
        part[(i >> 2) & 255] = part[(i >> 2) & 255] + (double)(v * v);
    }
    const float var = (float)(fold_d(part, 256) / (double)n);
    const float scale = 1.0f / sqrtf(var + eps);
    for (int i = 0; i < n; ++i) {
        float v = y[i] * scale;
        v = v * w[i];
        y[i] = v + b[i];
    }
}

/* ------------------------------------------------------------------------------------ */
/* sinusoid (lm.h:102-116)                                                              */
/* ------------------------------------------------------------------------------------ */
REF_API void ref_sin_positions(int first, int n, int dim, int pos_denominator, float max_period, float* out) {
    const int half = dim / 2;
    const double denom = (double)pos_denominator;
    for (int t = 0; t < n; ++t) {
        float* dst = out + (size_t)t * dim;
        const double pos = (double)(first + t);
        for (int i = 0; i < half; ++i) {
            const double phase = pos / pow((double)max_period, (double)i / denom);
            dst[i] = (float)cos(phase);
            dst[half + i] = (float)sin(phase);
        }
    }
}

/* ------------------------------------------------------------------------------------ */
/* attention: one query against keys [0,u) (nn.h:186-191)                               */
/* ------------------------------------------------------------------------------------ */
#define ATT_CHUNK 64    /* keys per attention chunk */
#define ATT_SLOTS 64    /* chunks of one attention (4096 keys) */

static inline float dot_qk(const float* q, const float* k, int hd) {
    float part[16];
    for (int l = 0; l < 16; ++l) part[l] = 0.0f;
    for (int i = 0; i < hd; ++i) part[(i >> 2) & 15] = fmaf(q[i], k[i], part[(i >> 2) & 15]);
    return fold_f(part, 16);
}

/* K: key j's row at K + j*k_stride (hd floats); V^T: dim d's row at VT + d*vt_stride, key j
   at + j. mask_row: additive, [u], or NULL. s: scratch [u]. u <= ATT_CHUNK * ATT_SLOTS.
   Keys in chunks of ATT_CHUNK (64). Per chunk c: its max m_c over the chunk's unmasked scores
   (a chunk whose keys are all masked is skipped), e_j = expf(s_j - m_c), the chunk sum S_c of
   the e_j in double (64-wide butterfly over the chunk's keys, zeros past its end), and o_c =
   sum_j e_j v_j per dim as 16 key-strided fmaf partials (key j -> partial j mod 16, increasing
   j) + butterfly. Then M = max m_c, w_c = exp((double)m_c - M) in double, total = the 64-wide
   butterfly of slots S_c * w_c (slot c, zeros for absent chunks), and out = sum over the
   chunks in order of fmaf(o_c, (float)(w_c / total), .) -- the softmax of nn.h:186-191 with
   its normalization applied per chunk. */
static void attend(const float* q, int hd, int u, const float* K, size_t k_stride, const float* VT,
                   size_t vt_stride, const float* mask_row, float scale, float* out, float* s) {
    const int nch = (u + ATT_CHUNK - 1) / ATT_CHUNK;
    if (nch > ATT_SLOTS || hd > 64) {   /* beyond every shape this oracle serves */
        for (int d = 0; d < hd; ++d) out[d] = NAN;
        return;
    }
    for (int j = 0; j < u; ++j) {
        float w = dot_qk(q, K + (size_t)j * k_stride, hd) * scale;
        if (mask_row) w = w + mask_row[j];
        s[j] = w;
    }
    float mc[ATT_SLOTS], oc[ATT_SLOTS][64];
    double sc[ATT_SLOTS];
    int live[ATT_SLOTS];
    for (int c = 0; c < nch; ++c) {
        const int j0 = c * ATT_CHUNK, j1 = j0 + ATT_CHUNK < u ? j0 + ATT_CHUNK : u;
        float m = -INFINITY;
        for (int j = j0; j < j1; ++j) m = m > s[j] ? m : s[j];
        live[c] = m != -INFINITY;
        mc[c] = m;
        if (!live[c]) continue;
        double part[ATT_CHUNK];
        for (int l = 0; l < ATT_CHUNK; ++l) {
            const int j = j0 + l;
            part[l] = 0.0;
            if (j < j1) { s[j] = ref_expf(s[j] - m); part[l] = (double)s[j]; }
        }
        sc[c] = fold_d(part, ATT_CHUNK);
        for (int d = 0; d < hd; ++d) {
            const float* vrow = VT + (size_t)d * vt_stride;
            float p16[16];
            for (int l = 0; l < 16; ++l) p16[l] = 0.0f;
            for (int mm = 0; mm < ATT_CHUNK / 16; ++mm)
                for (int g = 0; g < 16; ++g) {
                    const int j = j0 + g + 16 * mm;
                    if (j < j1) p16[g] = fmaf(s[j], vrow[j], p16[g]);
                }
            oc[c][d] = fold_f(p16, 16);
        }
    }
    float M = -INFINITY;
    for (int c = 0; c < nch; ++c) if (live[c]) M = M > mc[c] ? M : mc[c];
    double w[ATT_SLOTS], slot[ATT_SLOTS];
    for (int c = 0; c < ATT_SLOTS; ++c) {
        slot[c] = 0.0;
        if (c < nch && live[c]) {
            w[c] = ref_exp((double)mc[c] - (double)M);
            slot[c] = sc[c] * w[c];
        }
    }
    const double total = fold_d(slot, ATT_SLOTS);
    float f[ATT_SLOTS];
    for (int c = 0; c < nch; ++c) if (live[c]) f[c] = (float)(w[c] / total);
    for (int d = 0; d < hd; ++d) {
        float r = 0.0f;
        for (int c = 0; c < nch; ++c) if (live[c]) r = fmaf(oc[c][d], f[c], r);
        out[d] = r;
    }
}

/* Exposed for the decode-attention tests: q [hd], K rows [u][hd], V^T [hd][vt_stride]. */
REF_API void ref_attend(const float* q, int hd, int u, const float* K, const float* VT, int vt_stride,
                        const float* mask_row, float scale, float* out) {
    float* s = (float*)malloc(sizeof(float) * (size_t)(u > 0 ? u : 1));
    attend(q, hd, u, K, (size_t)hd, VT, (size_t)vt_stride, mask_row, scale, out, s);
    free(s);
}

/* ------------------------------------------------------------------------------------ */
/* model                                                                                */
/* ------------------------------------------------------------------------------------ */
typedef struct {
    int dim, layers, heads, head_dim, ff_dim, cond_dim, n_q, card, special_token_id, pos_denominator;
    float max_period, norm_eps, cfg_coef;
} ref_config;

typedef struct {
    const char* name;
    int type;
    int64_t ne0, ne1;
    const void* data;
} ref_tensor;

typedef struct {
    const char* target;     /* base tensor name, e.g. "lm.3.self.qkv.weight" */
    const float* A;         /* ggml [in, rank]: rank rows of in floats */
    const float* B;         /* ggml [rank, out]: out rows of rank floats */
    const float* magnitude; /* [out] or NULL */
    int rank;
    float alpha, strength;
} ref_adapter_tensor;

enum { P_QKV, P_OUT, P_CQ, P_CKV, P_COUT, P_FF0, P_FF2, P_COUNT };
static const char* PROJ_NAME[P_COUNT] = {"self.qkv", "self.out", "cross.q", "cross.kv", "cross.out", "ff.0", "ff.2"};

typedef struct {
    mat_t w[P_COUNT];
    adapter_t* ad[P_COUNT];
    const float *n1w, *n1b, *ncw, *ncb, *n2w, *n2b;
} layer_t;

typedef struct {
    ref_config c;
    mat_t emb[8], head[8], cond_proj;
    const float *cond_proj_b, *out_w, *out_b;
    layer_t* L;
    adapter_t* adapters;
    int n_adapters;
} ref_model;

static const ref_tensor* find_tensor(const ref_tensor* t, int n, const char* name) {
    for (int i = 0; i < n; ++i)
        if (strcmp(t[i].name, name) == 0) return &t[i];
    return NULL;
}

static int get_mat(const ref_tensor* t, int n, const char* name, int in, int out, mat_t* m) {
    const ref_tensor* x = find_tensor(t, n, name);
    if (!x) { snprintf(g_err, sizeof g_err, "missing tensor %s", name); return -1; }
    if (x->ne0 != in || x->ne1 != out) { snprintf(g_err, sizeof g_err, "bad shape for %s", name); return -1; }
    if (x->type != T_F32 && x->type != T_F16 && x->type != T_Q8_0 && x->type != T_Q4_0) {
        snprintf(g_err, sizeof g_err, "unsupported type for %s", name); return -1;
    }
    if ((x->type == T_Q8_0 || x->type == T_Q4_0) && in % 32) { snprintf(g_err, sizeof g_err, "%s: ne0 %% 32", name); return -1; }
    m->type = x->type; m->in = in; m->out = out; m->row_bytes = row_bytes_of(x->type, in);
    m->data = (const uint8_t*)x->data;
    return 0;
}
static const float* get_vec(const ref_tensor* t, int n, const char* name, int len) {
    const ref_tensor* x = find_tensor(t, n, name);
    if (!x || x->type != T_F32 || x->ne0 != len) { snprintf(g_err, sizeof g_err, "missing or bad f32 vector %s", name); return NULL; }
    return (const float*)x->data;
}

/* Row of a matrix dequantized to f32 (ggml get_rows / dequantize_row_*). */
static void dequant_row(const mat_t* m, int r, float* out) {
    const uint8_t* row = m->data + (size_t)r * m->row_bytes;
    if (m->type == T_F32) memcpy(out, row, sizeof(float) * (size_t)m->in);
    else if (m->type == T_F16) for (int i = 0; i < m->in; ++i) out[i] = f16at(row + 2 * i);
    else if (m->type == T_Q8_0)
        for (int b = 0; b < m->in / 32; ++b) {
            const float d = f16at(row + b * 34);
            const int8_t* q = (const int8_t*)(row + b * 34 + 2);
            for (int j = 0; j < 32; ++j) out[b * 32 + j] = (float)q[j] * d;
        }
    else
        for (int b = 0; b < m->in / 32; ++b) {
            const float d = f16at(row + b * 18);
            const uint8_t* q = row + b * 18 + 2;
            for (int j = 0; j < 16; ++j) {
                out[b * 32 + j] = (float)((int)(q[j] & 15) - 8) * d;
                out[b * 32 + j + 16] = (float)((int)(q[j] >> 4) - 8) * d;
            }
        }
}

REF_API void ref_model_destroy(ref_model* m) {
    if (!m) return;
    if (m->adapters)
        for (int i = 0; i < m->n_adapters; ++i) { free(m->adapters[i].base_norm_sq); free(m->adapters[i].norm); }
    free(m->adapters);
    free(m->L);
    free(m);
}

/* Model from ggml-named tensors (the GGUF contract of lm.h:60-90 and the converter's
   names). adapters: optional LoRA / DoRA-rows per projection (lora.h:113-176). */
REF_API ref_model* ref_model_create(const ref_config* cfg, const ref_tensor* t, int n,
                                    const ref_adapter_tensor* ads, int n_ads) {
    ref_model* m = (ref_model*)calloc(1, sizeof *m);
    m->c = *cfg;
    const ref_config* c = cfg;
    if (c->dim != c->heads * c->head_dim) { set_err("LM dim does not equal heads * head_dim"); free(m); return NULL; }
    if (c->special_token_id != c->card) { set_err("special_token_id should be card"); free(m); return NULL; }
    if (c->n_q > 8 || c->n_q <= 0) { set_err("n_q out of range"); free(m); return NULL; }
    char name[128];
    m->L = (layer_t*)calloc((size_t)c->layers, sizeof(layer_t));
    for (int q = 0; q < c->n_q; ++q) {
        snprintf(name, sizeof name, "lm.emb.%d.weight", q);
        if (get_mat(t, n, name, c->dim, c->card + 1, &m->emb[q])) goto fail;
        snprintf(name, sizeof name, "lm.head.%d.weight", q);
        if (get_mat(t, n, name, c->dim, c->card, &m->head[q])) goto fail;
    }
    if (get_mat(t, n, "lm.cond_proj.weight", c->cond_dim, c->dim, &m->cond_proj)) goto fail;
    if (!(m->cond_proj_b = get_vec(t, n, "lm.cond_proj.bias", c->dim))) goto fail;
    if (!(m->out_w = get_vec(t, n, "lm.out_norm.weight", c->dim))) goto fail;
    if (!(m->out_b = get_vec(t, n, "lm.out_norm.bias", c->dim))) goto fail;
    for (int i = 0; i < c->layers; ++i) {
        layer_t* L = &m->L[i];
        const int ins[P_COUNT] = {c->dim, c->dim, c->dim, c->dim, c->dim, c->dim, c->ff_dim};
        const int outs[P_COUNT] = {3 * c->dim, c->dim, c->dim, 2 * c->dim, c->dim, c->ff_dim, c->dim};
        for (int p = 0; p < P_COUNT; ++p) {
            snprintf(name, sizeof name, "lm.%d.%s.weight", i, PROJ_NAME[p]);
            if (get_mat(t, n, name, ins[p], outs[p], &L->w[p])) goto fail;
        }
        const char* norms[3] = {"norm1", "norm_cross", "norm2"};
        const float** ws[3] = {&L->n1w, &L->ncw, &L->n2w};
        const float** bs[3] = {&L->n1b, &L->ncb, &L->n2b};
        for (int k = 0; k < 3; ++k) {
            snprintf(name, sizeof name, "lm.%d.%s.weight", i, norms[k]);
            if (!(*ws[k] = get_vec(t, n, name, c->dim))) goto fail;
            snprintf(name, sizeof name, "lm.%d.%s.bias", i, norms[k]);
            if (!(*bs[k] = get_vec(t, n, name, c->dim))) goto fail;
        }
    }
    if (n_ads > 0) {
        m->adapters = (adapter_t*)calloc((size_t)n_ads, sizeof(adapter_t));
        m->n_adapters = n_ads;
        for (int a = 0; a < n_ads; ++a) {
            const ref_adapter_tensor* s = &ads[a];
            int li = -1, pi = -1;
            for (int i = 0; i < c->layers && li < 0; ++i)
                for (int p = 0; p < P_COUNT; ++p) {
                    snprintf(name, sizeof name, "lm.%d.%s.weight", i, PROJ_NAME[p]);
                    if (strcmp(name, s->target) == 0) { li = i; pi = p; break; }
                }
            if (li < 0) { snprintf(g_err, sizeof g_err, "unsupported MusicGen adapter target: %s", s->target); goto fail; }
            if (s->rank <= 0 || !isfinite(s->alpha) || s->alpha <= 0 || !isfinite(s->strength)) {
                set_err("invalid adapter rank, alpha or strength"); goto fail;
            }
            adapter_t* ad = &m->adapters[a];
            const mat_t* W = &m->L[li].w[pi];
            ad->A = s->A; ad->B = s->B; ad->magnitude = s->magnitude; ad->rank = s->rank;
            ad->scale = (s->magnitude ? 1.0f : s->strength) * s->alpha / (float)s->rank;   /* lora.h:142 */
            ad->strength = s->magnitude ? s->strength : 1.0f;
            const size_t nA = (size_t)s->rank * W->in, nB = (size_t)W->out * s->rank;
            for (size_t k = 0; k < nA; ++k) if (!isfinite(s->A[k])) { set_err("nonfinite adapter tensor"); goto fail; }
            for (size_t k = 0; k < nB; ++k) if (!isfinite(s->B[k])) { set_err("nonfinite adapter tensor"); goto fail; }
            if (s->magnitude) {
                for (int r = 0; r < W->out; ++r) if (!isfinite(s->magnitude[r])) { set_err("nonfinite adapter tensor"); goto fail; }
                /* DoRA rows: ||W_r||^2 from the dequantized base (the reference accepts only
                   F16/F32 bases, lora.h:11-13; a quantized base uses its dequantized rows),
                   then ||W + sBA||^2 = ||W||^2 + 2s<W,BA> + s^2||BA||^2 per row, all fixed
                   for the adapter's life. */
                ad->base_norm_sq = (float*)malloc(sizeof(float) * (size_t)W->out);
                ad->norm = (float*)malloc(sizeof(float) * (size_t)W->out);
                int bad = 0;
                #pragma omp parallel for schedule(static) reduction(|:bad)
                for (int r = 0; r < W->out; ++r) {
                    float* wr = (float*)malloc(sizeof(float) * (size_t)W->in);
                    float* ba = (float*)malloc(sizeof(float) * (size_t)W->in);
                    dequant_row(W, r, wr);
                    double sum = (double)W->in * 1e-12;
                    for (int i = 0; i < W->in; ++i) { if (!isfinite(wr[i])) bad = 1; sum += (double)wr[i] * wr[i]; }
                    ad->base_norm_sq[r] = (float)sum;
                    for (int i = 0; i < W->in; ++i) {
                        double acc = 0.0;
                        for (int k = 0; k < s->rank; ++k) acc += (double)s->B[(size_t)r * s->rank + k] * s->A[(size_t)k * W->in + i];
                        ba[i] = (float)acc;
                    }
                    double t2 = 0.0, t3 = 0.0;
                    for (int i = 0; i < W->in; ++i) { t2 += (double)wr[i] * ba[i]; t3 += (double)ba[i] * ba[i]; }
                    const double nsq = (double)ad->base_norm_sq[r] + 2.0 * ad->scale * t2 + (double)ad->scale * ad->scale * t3;
                    ad->norm[r] = (float)sqrt(nsq);
                    free(wr); free(ba);
                }
                if (bad) { set_err("nonfinite DoRA base weight"); goto fail; }
            }
            m->L[li].ad[pi] = ad;
        }
    }
    return m;
fail:
    ref_model_destroy(m);
    return NULL;
}

/* ------------------------------------------------------------------------------------ */
/* decoder (pipeline.cpp:36-195)                                                        */
/* ------------------------------------------------------------------------------------ */
typedef struct {
    const ref_model* m;
    int capacity, n_seq, cross, n_ctx, used, forwards, recompute_cross_kv;
    float* K;        /* per layer: [n_seq][H][cap][hd]  (ggml [hd, cap, H, n_seq]) */
    float* VT;       /* per layer: [n_seq][H][hd][cap]  (ggml [cap, hd, H, n_seq]) */
    float* context;  /* [n_seq][n_ctx][dim]; stream 1 stays zero */
    float* cross_kv; /* hoisted: per layer [n_seq][n_ctx][2*dim] */
} ref_decoder;

REF_API void ref_decoder_destroy(ref_decoder* d) {
    if (!d) return;
    free(d->K); free(d->VT); free(d->context); free(d->cross_kv); free(d);
}

static void cross_kv_layer(const ref_decoder* d, int layer, float* out /* [n_seq][n_ctx][2d] */) {
    const ref_model* m = d->m;
    matmul(&m->L[layer].w[P_CKV], m->L[layer].ad[P_CKV], d->context, d->n_seq * d->n_ctx, out);
}

/* t5_hidden: [n_ctx][cond_dim] (ggml [cond_dim, n_ctx]). cross: guidance on (n_seq 2) or
   off; capacity: the pattern length S. recompute_cross_kv: 1 repeats the reference's per-step
   cross.kv projection (lm.h:184), 0 projects it once; both give the same numbers. */
REF_API ref_decoder* ref_decoder_create(const ref_model* m, int capacity, int n_seq, const float* t5_hidden,
                                        int n_ctx, int cross, int recompute_cross_kv) {
    const ref_config* c = &m->c;
    if (capacity <= 0 || n_seq <= 0) { set_err("the kv cache needs positive dimensions"); return NULL; }
    ref_decoder* d = (ref_decoder*)calloc(1, sizeof *d);
    d->m = m; d->capacity = capacity; d->n_seq = n_seq; d->cross = cross;
    d->recompute_cross_kv = recompute_cross_kv;
    const size_t per = (size_t)n_seq * c->heads * capacity * c->head_dim;
    d->K = (float*)calloc(per * c->layers, sizeof(float));
    d->VT = (float*)calloc(per * c->layers, sizeof(float));
    if (!d->K || !d->VT) { set_err("failed to allocate the kv cache"); ref_decoder_destroy(d); return NULL; }
    if (cross) {
        if (n_ctx <= 0) { set_err("the conditioning has no tokens"); ref_decoder_destroy(d); return NULL; }
        d->n_ctx = n_ctx;
        d->context = (float*)calloc((size_t)n_seq * n_ctx * c->dim, sizeof(float));
        /* lm.cond_proj . t5 + bias into stream 0 only (pipeline.cpp:144-180). */
        matmul(&m->cond_proj, NULL, t5_hidden, n_ctx, d->context);
        for (int t = 0; t < n_ctx; ++t)
            for (int i = 0; i < c->dim; ++i) d->context[(size_t)t * c->dim + i] = d->context[(size_t)t * c->dim + i] + m->cond_proj_b[i];
        if (!recompute_cross_kv) {
            d->cross_kv = (float*)malloc(sizeof(float) * (size_t)c->layers * n_seq * n_ctx * 2 * c->dim);
            for (int l = 0; l < c->layers; ++l)
                cross_kv_layer(d, l, d->cross_kv + (size_t)l * n_seq * n_ctx * 2 * c->dim);
        }
    }
    return d;
}

REF_API int ref_decoder_used(const ref_decoder* d) { return d->used; }
REF_API void ref_decoder_reset(ref_decoder* d) { d->used = 0; }
REF_API size_t ref_decoder_cache_bytes(const ref_decoder* d) {
    const ref_config* c = &d->m->c;
    return (size_t)c->layers * 2 * c->head_dim * d->capacity * c->heads * d->n_seq * sizeof(float);
}

/* Decoder::forward: n_tokens steps at codebook-major ids [n_q][n_tokens]; writes the last
   position's logits [n_seq][n_q][card]. Returns 0, or -1 with ref_last_error(). */
REF_API int ref_forward(ref_decoder* d, const int32_t* ids, int n_tokens, float* logits) {
    const ref_model* m = d->m;
    const ref_config* c = &m->c;
    const int D = c->dim, H = c->heads, hd = c->head_dim, N = d->n_seq, T = n_tokens, F = c->ff_dim;
    if (T <= 0) { set_err("n_tokens must be positive"); return -1; }
    if (T > 1 && d->used != 0) { set_err("multi-token forwards are only supported as a prefill"); return -1; }
    if (d->used + T > d->capacity) { set_err("kv cache overflow: the sequence is longer than its capacity"); return -1; }
    for (int q = 0; q < c->n_q; ++q)
        for (int t = 0; t < T; ++t) {
            const int id = ids[(size_t)q * T + t];
            if (id < 0 || id > c->card) { set_err("token id out of range"); return -1; }
        }
    const int cols = T * N;
    /* x: [t][n][D] -> column index t*N + n */
    float* x = (float*)malloc(sizeof(float) * (size_t)cols * D);
    float* h = (float*)malloc(sizeof(float) * (size_t)cols * D);
    float* big = (float*)malloc(sizeof(float) * (size_t)cols * (3 * D > F ? 3 * D : F));
    float* o = (float*)malloc(sizeof(float) * (size_t)cols * D);
    float* y = (float*)malloc(sizeof(float) * (size_t)cols * D);
    float* pos = (float*)malloc(sizeof(float) * (size_t)T * D);
    float* row = (float*)malloc(sizeof(float) * (size_t)D);
    ref_sin_positions(d->used, T, D, c->pos_denominator, c->max_period, pos);
    /* Embedding sum then + pos (lm.h:231-240); broadcast across streams. */
    for (int t = 0; t < T; ++t) {
        float* e = y;  /* [D] */
        for (int q = 0; q < c->n_q; ++q) {
            dequant_row(&m->emb[q], ids[(size_t)q * T + t], row);
            for (int i = 0; i < D; ++i) e[i] = q == 0 ? row[i] : e[i] + row[i];
        }
        for (int n = 0; n < N; ++n)
            for (int i = 0; i < D; ++i) x[((size_t)t * N + n) * D + i] = pos[(size_t)t * D + i] + e[i];
    }
    const int u = d->used + T;                          /* keys in the history view */
    const float scale = 1.0f / sqrtf((float)hd);
    float* mask = NULL;
    if (T > 1) {                                        /* pipeline.cpp:115-121 */
        mask = (float*)malloc(sizeof(float) * (size_t)T * T);
        for (int qi = 0; qi < T; ++qi)
            for (int kj = 0; kj < T; ++kj) mask[(size_t)qi * T + kj] = kj > qi ? -INFINITY : 0.0f;
    }
    const size_t per_layer = (size_t)N * H * d->capacity * hd;
    float* ckv_step = NULL;
    if (d->cross && d->recompute_cross_kv) ckv_step = (float*)malloc(sizeof(float) * (size_t)N * d->n_ctx * 2 * D);
    for (int l = 0; l < c->layers; ++l) {
        const layer_t* L = &m->L[l];
        float* Kl = d->K + (size_t)l * per_layer;
        float* Vl = d->VT + (size_t)l * per_layer;
        /* --- self-attention --- */
        for (int col = 0; col < cols; ++col) ref_layer_norm(x + (size_t)col * D, D, L->n1w, L->n1b, c->norm_eps, h + (size_t)col * D);
        matmul(&L->w[P_QKV], L->ad[P_QKV], h, cols, big);           /* [col][3D] */
        for (int t = 0; t < T; ++t)
            for (int n = 0; n < N; ++n) {
                const float* qkv = big + ((size_t)t * N + n) * 3 * D;
                for (int hh = 0; hh < H; ++hh) {
                    float* kd = Kl + (((size_t)n * H + hh) * d->capacity + (d->used + t)) * hd;
                    for (int i = 0; i < hd; ++i) kd[i] = qkv[D + hh * hd + i];
                    float* vd = Vl + ((size_t)n * H + hh) * hd * d->capacity + (d->used + t);
                    for (int i = 0; i < hd; ++i) vd[(size_t)i * d->capacity] = qkv[2 * D + hh * hd + i];
                }
            }
        #pragma omp parallel
        {
            float* s = (float*)malloc(sizeof(float) * (size_t)u);
            #pragma omp for collapse(3) schedule(static)
            for (int t = 0; t < T; ++t)
                for (int n = 0; n < N; ++n)
                    for (int hh = 0; hh < H; ++hh) {
                        const float* q = big + ((size_t)t * N + n) * 3 * D + hh * hd;
                        const float* Kh = Kl + ((size_t)n * H + hh) * d->capacity * hd;
                        const float* Vh = Vl + ((size_t)n * H + hh) * hd * d->capacity;
                        attend(q, hd, u, Kh, (size_t)hd, Vh, (size_t)d->capacity, mask ? mask + (size_t)t * T : NULL,
                               scale, o + ((size_t)t * N + n) * D + hh * hd, s);
                    }
            free(s);
        }
        matmul(&L->w[P_OUT], L->ad[P_OUT], o, cols, y);
        for (size_t i = 0; i < (size_t)cols * D; ++i) x[i] = x[i] + y[i];
        /* --- cross-attention (lm.h:181-199) --- */
        if (d->cross) {
            for (int col = 0; col < cols; ++col) ref_layer_norm(x + (size_t)col * D, D, L->ncw, L->ncb, c->norm_eps, h + (size_t)col * D);
            matmul(&L->w[P_CQ], L->ad[P_CQ], h, cols, big);         /* [col][D] */
            const float* ckv;
            if (d->recompute_cross_kv) { cross_kv_layer(d, l, ckv_step); ckv = ckv_step; }
            else ckv = d->cross_kv + (size_t)l * N * d->n_ctx * 2 * D;
            const int nc = d->n_ctx;
            #pragma omp parallel
            {
                float* s = (float*)malloc(sizeof(float) * (size_t)nc);
                float* vt = (float*)malloc(sizeof(float) * (size_t)hd * nc);
                float* kr = (float*)malloc(sizeof(float) * (size_t)nc * hd);
                #pragma omp for collapse(3) schedule(static)
                for (int t = 0; t < T; ++t)
                    for (int n = 0; n < N; ++n)
                        for (int hh = 0; hh < H; ++hh) {
                            const float* base = ckv + (size_t)n * nc * 2 * D;
                            for (int j = 0; j < nc; ++j)
                                for (int i = 0; i < hd; ++i) {
                                    kr[(size_t)j * hd + i] = base[(size_t)j * 2 * D + hh * hd + i];
                                    vt[(size_t)i * nc + j] = base[(size_t)j * 2 * D + D + hh * hd + i];
                                }
                            attend(big + ((size_t)t * N + n) * D + hh * hd, hd, nc, kr, (size_t)hd, vt, (size_t)nc, NULL,
                                   scale, o + ((size_t)t * N + n) * D + hh * hd, s);
                        }
                free(s); free(vt); free(kr);
            }
            matmul(&L->w[P_COUT], L->ad[P_COUT], o, cols, y);
            for (size_t i = 0; i < (size_t)cols * D; ++i) x[i] = x[i] + y[i];
        }
        /* --- feed-forward --- */
        for (int col = 0; col < cols; ++col) ref_layer_norm(x + (size_t)col * D, D, L->n2w, L->n2b, c->norm_eps, h + (size_t)col * D);
        matmul(&L->w[P_FF0], L->ad[P_FF0], h, cols, big);           /* [col][F] */
        for (size_t i = 0; i < (size_t)cols * F; ++i) big[i] = ref_gelu_erf(big[i]);
        matmul(&L->w[P_FF2], L->ad[P_FF2], big, cols, y);
        for (size_t i = 0; i < (size_t)cols * D; ++i) x[i] = x[i] + y[i];
    }
    /* Last position -> out_norm -> heads (lm.h:248-258). */
    for (int n = 0; n < N; ++n)
        ref_layer_norm(x + ((size_t)(T - 1) * N + n) * D, D, m->out_w, m->out_b, c->norm_eps, h + (size_t)n * D);
    for (int q = 0; q < c->n_q; ++q) {
        matmul(&m->head[q], NULL, h, N, big);                       /* [n][card] */
        for (int n = 0; n < N; ++n)
            memcpy(logits + ((size_t)n * c->n_q + q) * c->card, big + (size_t)n * c->card, sizeof(float) * (size_t)c->card);
    }
    d->used += T;
    d->forwards += 1;
    free(x); free(h); free(big); free(o); free(y); free(pos); free(row); free(mask); free(ckv_step);
    return 0;
}

/* ------------------------------------------------------------------------------------ */
/* RNG (rng.h:15-33): std::mt19937 seeded with (uint32)seed                              */
/* ------------------------------------------------------------------------------------ */
typedef struct { uint32_t mt[624]; int idx; } ref_rng;

REF_API void ref_rng_seed(ref_rng* r, uint64_t seed) {
    r->mt[0] = (uint32_t)seed;
    for (int i = 1; i < 624; ++i) r->mt[i] = 1812433253u * (r->mt[i - 1] ^ (r->mt[i - 1] >> 30)) + (uint32_t)i;
    r->idx = 624;
}
REF_API uint32_t ref_rng_next(ref_rng* r) {
    if (r->idx >= 624) {
        for (int i = 0; i < 624; ++i) {
            const uint32_t y = (r->mt[i] & 0x80000000u) | (r->mt[(i + 1) % 624] & 0x7fffffffu);
            r->mt[i] = r->mt[(i + 397) % 624] ^ (y >> 1) ^ ((y & 1u) ? 0x9908b0dfu : 0u);
        }
        r->idx = 0;
    }
    uint32_t y = r->mt[r->idx++];
    y ^= y >> 11;
    y ^= (y << 7) & 0x9d2c5680u;
    y ^= (y << 15) & 0xefc60000u;
    y ^= y >> 18;
    return y;
}
REF_API float ref_rng_uniform(ref_rng* r) {
    return ((float)(ref_rng_next(r) >> 8) + 0.5f) * (1.0f / 16777216.0f);
}
REF_API size_t ref_rng_size(void) { return sizeof(ref_rng); }

/* ------------------------------------------------------------------------------------ */
/* sampling (sampling.h:32-105)                                                         */
/* ------------------------------------------------------------------------------------ */
REF_API int ref_argmax(const float* x, int n) {
    int best = 0;
    for (int i = 1; i < n; ++i) if (x[i] > x[best]) best = i;
    return best;
}
REF_API void ref_softmax_into(const float* logits, int n, float temperature, float* probs) {
    float peak = logits[0];
    for (int i = 1; i < n; ++i) peak = peak < logits[i] ? logits[i] : peak;
    double total = 0.0;
    for (int i = 0; i < n; ++i) {
        const double e = exp(((double)logits[i] - peak) / temperature);
        probs[i] = (float)e;
        total += e;
    }
    const float inv = (float)(1.0 / total);
    for (int i = 0; i < n; ++i) probs[i] *= inv;
}
/* softmax_into with the GPU sampler's exp routine (ref_exp, the same Cody-Waite + Taylor
   steps as the kernel's) in place of libm's exp: the tests count the rows where the two
   give different float probabilities. */
REF_API void ref_softmax_into_devexp(const float* logits, int n, float temperature, float* probs) {
    float peak = logits[0];
    for (int i = 1; i < n; ++i) peak = peak < logits[i] ? logits[i] : peak;
    double total = 0.0;
    for (int i = 0; i < n; ++i) {
        const double e = ref_exp(((double)logits[i] - peak) / temperature);
        probs[i] = (float)e;
        total += e;
    }
    const float inv = (float)(1.0 / total);
    for (int i = 0; i < n; ++i) probs[i] *= inv;
}
/* Rows [rows][n]: how many rows' probabilities differ between libm's exp and ref_exp, and how
   many of the exp values differ at all (in double). */
REF_API void ref_softmax_exp_compare(const float* logits, int n, int rows, float temperature, long long* row_diff,
                                     long long* exp_diff) {
    long long rd = 0, ed = 0;
    #pragma omp parallel for reduction(+:rd, ed) schedule(static)
    for (int r = 0; r < rows; ++r) {
        const float* x = logits + (size_t)r * n;
        float* a = (float*)malloc(sizeof(float) * (size_t)n);
        float* b = (float*)malloc(sizeof(float) * (size_t)n);
        ref_softmax_into(x, n, temperature, a);
        ref_softmax_into_devexp(x, n, temperature, b);
        if (memcmp(a, b, sizeof(float) * (size_t)n) != 0) ++rd;
        float peak = x[0];
        for (int i = 1; i < n; ++i) peak = peak < x[i] ? x[i] : peak;
        for (int i = 0; i < n; ++i) {
            const double t = ((double)x[i] - peak) / temperature;
            if (exp(t) != ref_exp(t)) ++ed;
        }
        free(a); free(b);
    }
    *row_diff = rd;
    *exp_diff = ed;
}
static int cmp_desc(const void* a, const void* b) {
    const float x = *(const float*)a, y = *(const float*)b;
    return x < y ? 1 : (x > y ? -1 : 0);
}
/* The cutoff is the k-th largest value counting repeats (what the reference's min-heap of
   the k largest holds at its top); everything below it is zeroed, ties survive. */
REF_API void ref_top_k_filter(float* probs, int n, int k) {
    if (k <= 0 || k >= n) return;
    float* s = (float*)malloc(sizeof(float) * (size_t)n);
    memcpy(s, probs, sizeof(float) * (size_t)n);
    qsort(s, (size_t)n, sizeof(float), cmp_desc);
    const float cutoff = s[k - 1];
    free(s);
    double total = 0.0;
    for (int i = 0; i < n; ++i) {
        if (probs[i] < cutoff) probs[i] = 0.0f;
        total += (double)probs[i];
    }
    const float inv = (float)(1.0 / total);
    for (int i = 0; i < n; ++i) probs[i] *= inv;
}
REF_API int ref_categorical(const float* w, int n, double total, ref_rng* rng) {
    if (!(total > 0.0)) return -1;
    const double target = (double)ref_rng_uniform(rng) * total;
    double acc = 0.0;
    for (int i = 0; i < n; ++i) {
        acc += (double)w[i];
        if (acc > target) return i;
    }
    return n - 1;
}
REF_API int ref_sample_top_k(const float* logits, int n, int k, float temperature, ref_rng* rng, float* scratch) {
    if (!(temperature > 0.0f)) return ref_argmax(logits, n);
    ref_softmax_into(logits, n, temperature, scratch);
    ref_top_k_filter(scratch, n, k);
    return ref_categorical(scratch, n, 1.0, rng);
}

/* ------------------------------------------------------------------------------------ */
/* delay pattern (pattern.h:31-115), delays 0..n_q-1                                     */
/* ------------------------------------------------------------------------------------ */
REF_API int ref_pattern_steps(int n_q, int timesteps) { return 1 + timesteps + (n_q - 1); }
static int timestep_at(int q, int s, int T) {
    if (s <= 0) return -1;
    const int t = s - 1 - q;
    return (t >= 0 && t < T) ? t : -1;
}
REF_API void ref_build_pattern(int n_q, int T, const int32_t* codes, int32_t special, int32_t* seq) {
    const int S = ref_pattern_steps(n_q, T);
    for (int q = 0; q < n_q; ++q)
        for (int s = 0; s < S; ++s) {
            const int t = timestep_at(q, s, T);
            seq[(size_t)q * S + s] = t >= 0 ? codes[(size_t)q * T + t] : special;
        }
}
REF_API void ref_revert_pattern(int n_q, int T, const int32_t* seq, int32_t special, int32_t* codes) {
    const int S = ref_pattern_steps(n_q, T);
    for (size_t i = 0; i < (size_t)n_q * T; ++i) codes[i] = special;
    for (int q = 0; q < n_q; ++q)
        for (int s = 0; s < S; ++s) {
            const int t = timestep_at(q, s, T);
            if (t >= 0) codes[(size_t)q * T + t] = seq[(size_t)q * S + s];
        }
}
REF_API void ref_pattern_mask(int n_q, int T, uint8_t* mask) {
    const int S = ref_pattern_steps(n_q, T);
    for (int q = 0; q < n_q; ++q)
        for (int s = 0; s < S; ++s) mask[(size_t)q * S + s] = timestep_at(q, s, T) >= 0 ? 1 : 0;
}

/* ------------------------------------------------------------------------------------ */
/* mg_generate (pipeline.cpp:199-314)                                                   */
/* ------------------------------------------------------------------------------------ */
typedef struct {
    int max_gen_len;
    int use_sampling;
    float temperature;
    int top_k;
    float cfg_coef;
    uint64_t seed;
} ref_gen_params;   /* GenerateParams (pipeline.h:25-34) */

typedef struct {
    size_t cache_bytes;
    int prefill_tokens, decode_steps, forwards;
    double prefill_seconds, decode_seconds;
} ref_report;       /* GenerateReport (pipeline.h:45-56), first_logits returned separately */

static double now_s(void) {
    struct timespec ts; clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

REF_API int ref_use_guidance(float cfg_coef, int description_empty) {
    return cfg_coef != 0.0f && !description_empty;
}

/* Timing samples of long prompts: with the flag set, ref_generate replaces the prompt's prefill
   forward by marking the caches as holding its positions (zero rows) and samples the first
   step from zero logits. Every decode step after it attends the same number of keys as in the
   real run, and its cost does not depend on the values, so a CPU timing sample of late decode
   steps no longer waits minutes for a prefill it does not time. Codes and logits are then
   meaningless: for timing only. */
static int g_timing_history = 0;
REF_API void ref_set_timing_history(int on) { g_timing_history = on; }

/* codes_out: [n_q][max_gen_len]; first_logits: [n_q][card]; step_logits (optional):
   [S-start][n_q][card] combined logits of every forward, for step-by-step comparison.
   max_forwards > 0 stops after that many forwards (a bounded timing sample); the codes
   past that point are then left unfilled and the final check is skipped. */
REF_API int ref_generate(const ref_model* m, const float* t5_hidden, int n_ctx, int description_empty,
                         const int32_t* prompt, int prompt_len, const ref_gen_params* p,
                         int recompute_cross_kv, int max_forwards,
                         int32_t* codes_out, float* first_logits, float* step_logits, ref_report* rep) {
    const ref_config* c = &m->c;
    const int K = c->n_q, T = p->max_gen_len;
    if (T <= 0) { set_err("max_gen_len must be positive"); return -1; }
    if (prompt_len < 0 || prompt_len >= T) { set_err("the prompt must be shorter than the generation"); return -1; }
    if (n_ctx <= 0) { set_err("the conditioning has no tokens"); return -1; }
    const int S = ref_pattern_steps(K, T);
    const int start = prompt_len + 1;
    int32_t* codes = (int32_t*)malloc(sizeof(int32_t) * (size_t)K * T);
    for (size_t i = 0; i < (size_t)K * T; ++i) codes[i] = -1;
    for (int q = 0; q < K; ++q)
        for (int t = 0; t < prompt_len; ++t) codes[(size_t)q * T + t] = prompt[(size_t)q * prompt_len + t];
    int32_t* seq = (int32_t*)malloc(sizeof(int32_t) * (size_t)K * S);
    ref_build_pattern(K, T, codes, c->special_token_id, seq);
    uint8_t* mask = (uint8_t*)malloc((size_t)K * S);
    ref_pattern_mask(K, T, mask);
    const int guided = ref_use_guidance(p->cfg_coef, description_empty);
    const int n_seq = guided ? 2 : 1;
    ref_decoder* dec = ref_decoder_create(m, S, n_seq, t5_hidden, n_ctx, guided, recompute_cross_kv);
    if (!dec) { free(codes); free(seq); free(mask); return -1; }
    ref_rng rng; ref_rng_seed(&rng, p->seed);
    float* out = (float*)malloc(sizeof(float) * (size_t)c->card * K * n_seq);
    float* combined = (float*)malloc(sizeof(float) * (size_t)c->card * K);
    float* scratch = (float*)malloc(sizeof(float) * (size_t)c->card);
    int32_t* feed = (int32_t*)malloc(sizeof(int32_t) * (size_t)K * S);
    rep->prefill_tokens = start;
    rep->decode_steps = S - start - 1;
    int previous = 0, rc = 0, done = 0;
    double t0 = now_s();
    for (int offset = start; offset < S; ++offset) {
        if (max_forwards > 0 && done >= max_forwards) break;
        const int nt = offset - previous;
        for (int q = 0; q < K; ++q) memcpy(feed + (size_t)q * nt, seq + (size_t)q * S + previous, sizeof(int32_t) * (size_t)nt);
        if (g_timing_history && offset == start) {
            dec->used = nt;
            dec->forwards += 1;
            memset(out, 0, sizeof(float) * (size_t)c->card * K * n_seq);
        } else if (ref_forward(dec, feed, nt, out)) { rc = -1; break; }
        ++done;
        const float* logits = out;
        if (guided) {
            const float* cl = out;
            const float* nl = out + (size_t)c->card * K;
            for (size_t i = 0; i < (size_t)c->card * K; ++i) combined[i] = nl[i] + (cl[i] - nl[i]) * p->cfg_coef;
            logits = combined;
        }
        if (offset == start && first_logits) memcpy(first_logits, logits, sizeof(float) * (size_t)c->card * K);
        if (step_logits) memcpy(step_logits + (size_t)(offset - start) * c->card * K, logits, sizeof(float) * (size_t)c->card * K);
        for (int q = 0; q < K; ++q) {
            const float* r = logits + (size_t)q * c->card;
            int token;
            if (!mask[(size_t)q * S + offset]) token = c->special_token_id;
            else if (p->use_sampling) token = ref_sample_top_k(r, c->card, p->top_k, p->temperature, &rng, scratch);
            else token = ref_argmax(r, c->card);
            if (token < 0) { set_err("categorical needs a positive total weight"); rc = -1; break; }
            int32_t* slot = &seq[(size_t)q * S + offset];
            if (*slot == -1) *slot = token;
        }
        if (rc) break;
        previous = offset;
        if (offset == start) { rep->prefill_seconds = now_s() - t0; t0 = now_s(); }
    }
    rep->decode_seconds = now_s() - t0;
    rep->forwards = dec->forwards;
    rep->cache_bytes = ref_decoder_cache_bytes(dec);
    if (!rc) {
        ref_revert_pattern(K, T, seq, c->special_token_id, codes_out);
        if (max_forwards <= 0)
            for (size_t i = 0; i < (size_t)K * T; ++i)
                if (codes_out[i] < 0 || codes_out[i] >= c->card) {
                    set_err("the generated sequence has a position the pattern never filled"); rc = -1; break;
                }
    }
    ref_decoder_destroy(dec);
    free(codes); free(seq); free(mask); free(out); free(combined); free(scratch); free(feed);
    return rc;
}

/* Bumped whenever a documented reduction order changes; fixtures record it. */
/* ------------------------------------------------------------------------------------ */
/* T5-base encoder (src/ac/t5.h:20-140, src/ac/conditioner.h:56-108)                     */
/* ------------------------------------------------------------------------------------ */
/* Conventions beyond the decode path's: rms_norm = mean of squares as a double sum
   (element i -> partial (i/4) mod 256 of (double)(x*x), 256-wide butterfly), then
   (x * (1.0f / sqrtf(mean + eps))) * w, each product rounded in f32 (ggml_rms_norm then
   ggml_mul). The learned position bias is added to the unscaled q.k score (t5.h:120-121:
   mul_mat, then add of bias + mask, the mask all zeros), soft_max and V as in attend(). ReLU
   maps everything not above zero to 0. */
typedef struct {
    int dim, layers, heads, head_dim, intermediate, vocab, relative_buckets, relative_max_distance;
    float eps;
} ref_t5_config;

/* transformers' T5Attention._relative_position_bucket, bidirectional (t5.h:46-61):
   relative position = key - query; the upper half of the buckets holds keys after the query;
   distances below a quarter of the buckets map one to one, longer ones logarithmically up to
   max_distance. The logarithm is taken in f32 as the reference does. */
REF_API int ref_t5_bucket(int relative_position, int num_buckets, int max_distance) {
    const int half = num_buckets / 2, exact = half / 2;
    const int base = relative_position > 0 ? half : 0;
    const int dist = relative_position < 0 ? -relative_position : relative_position;
    if (dist < exact) return base + dist;
    int far = exact;
    const float span = logf((float)max_distance / (float)exact);
    if (span > 0.0f) far += (int)(logf((float)dist / (float)exact) / span * (float)(half - exact));
    return base + (far < half - 1 ? far : half - 1);
}

static void rms_norm(const float* x, int n, const float* w, float eps, float* y) {
    double part[256];
    for (int l = 0; l < 256; ++l) part[l] = 0.0;
    for (int i = 0; i < n; ++i) part[(i >> 2) & 255] = part[(i >> 2) & 255] + (double)(x[i] * x[i]);
    const float mean = (float)(fold_d(part, 256) / (double)n);
    const float scale = 1.0f / sqrtf(mean + eps);
    for (int i = 0; i < n; ++i) {
        const float v = x[i] * scale;
        y[i] = v * w[i];
    }
}

REF_API void ref_rms_norm(const float* x, int n, const float* w, float eps, float* y) { rms_norm(x, n, w, eps, y); }

/* last_hidden_state [seq][dim] of ids [seq] (t5_encode, t5.h:85-140, as encode_prompt runs it:
   no padding, an all-zero mask). Returns 0, or -1 with ref_last_error. */
REF_API int ref_t5_encode(const ref_t5_config* c, const ref_tensor* t, int n, const int32_t* ids, int seq,
                          float* out) {
    const int D = c->dim, H = c->heads, hd = c->head_dim, inner = c->heads * c->head_dim, F = c->intermediate;
    if (seq <= 0) { set_err("no tokens"); return -1; }
    mat_t emb, rel;
    if (get_mat(t, n, "te.embed.weight", D, c->vocab, &emb) ||
        get_mat(t, n, "te.relative_attention_bias.weight", H, c->relative_buckets, &rel))
        return -1;
    const float* fnorm = get_vec(t, n, "te.norm.weight", D);
    if (!fnorm) return -1;
    for (int i = 0; i < seq; ++i)
        if (ids[i] < 0 || ids[i] >= c->vocab) { set_err("token id out of range"); return -1; }
    float* x = (float*)malloc(sizeof(float) * (size_t)seq * D);
    float* h = (float*)malloc(sizeof(float) * (size_t)seq * (D > inner ? D : inner));
    float* q = (float*)malloc(sizeof(float) * (size_t)seq * inner);
    float* k = (float*)malloc(sizeof(float) * (size_t)seq * inner);
    float* v = (float*)malloc(sizeof(float) * (size_t)seq * inner);
    float* vt = (float*)malloc(sizeof(float) * (size_t)inner * seq);
    float* o = (float*)malloc(sizeof(float) * (size_t)seq * inner);
    float* y = (float*)malloc(sizeof(float) * (size_t)seq * D);
    float* f = (float*)malloc(sizeof(float) * (size_t)seq * F);
    float* bias = (float*)malloc(sizeof(float) * (size_t)H * seq * seq);
    float* rowbuf = (float*)malloc(sizeof(float) * (size_t)(D > H ? D : H));
    float* sc = (float*)malloc(sizeof(float) * (size_t)seq);
    int rc = -1;
    for (int i = 0; i < seq; ++i) dequant_row(&emb, ids[i], x + (size_t)i * D);
    /* bias[h][q][k] = table[bucket(k - q)][h] + 0 (the zero mask added, t5.h:100) */
    for (int qi = 0; qi < seq; ++qi)
        for (int ki = 0; ki < seq; ++ki) {
            dequant_row(&rel, ref_t5_bucket(ki - qi, c->relative_buckets, c->relative_max_distance), rowbuf);
            for (int hh = 0; hh < H; ++hh) bias[((size_t)hh * seq + qi) * seq + ki] = rowbuf[hh] + 0.0f;
        }
    for (int l = 0; l < c->layers; ++l) {
        char name[96];
        mat_t wq, wk, wv, wo, wi, w2;
        const float *an, *fn;
#define T5M(field, stem, in_, out_) \
        snprintf(name, sizeof name, "te.%d." stem ".weight", l); \
        if (get_mat(t, n, name, in_, out_, &field)) goto done;
        T5M(wq, "q", D, inner) T5M(wk, "k", D, inner) T5M(wv, "v", D, inner) T5M(wo, "o", inner, D)
        T5M(wi, "wi", D, F) T5M(w2, "wo", F, D)
#undef T5M
        snprintf(name, sizeof name, "te.%d.attn_norm.weight", l);
        if (!(an = get_vec(t, n, name, D))) goto done;
        snprintf(name, sizeof name, "te.%d.ffn_norm.weight", l);
        if (!(fn = get_vec(t, n, name, D))) goto done;
        for (int i = 0; i < seq; ++i) rms_norm(x + (size_t)i * D, D, an, c->eps, h + (size_t)i * D);
        matmul(&wq, NULL, h, seq, q);
        matmul(&wk, NULL, h, seq, k);
        matmul(&wv, NULL, h, seq, v);
        for (int j = 0; j < seq; ++j)
            for (int d = 0; d < inner; ++d) vt[(size_t)d * seq + j] = v[(size_t)j * inner + d];
        for (int hh = 0; hh < H; ++hh)
            for (int qi = 0; qi < seq; ++qi)
                attend(q + (size_t)qi * inner + hh * hd, hd, seq, k + hh * hd, (size_t)inner,
                       vt + (size_t)hh * hd * seq, (size_t)seq, bias + ((size_t)hh * seq + qi) * seq, 1.0f,
                       o + (size_t)qi * inner + hh * hd, sc);
        matmul(&wo, NULL, o, seq, y);
        for (size_t i = 0; i < (size_t)seq * D; ++i) x[i] = x[i] + y[i];
        for (int i = 0; i < seq; ++i) rms_norm(x + (size_t)i * D, D, fn, c->eps, h + (size_t)i * D);
        matmul(&wi, NULL, h, seq, f);
        for (size_t i = 0; i < (size_t)seq * F; ++i) f[i] = f[i] > 0.0f ? f[i] : 0.0f;
        matmul(&w2, NULL, f, seq, y);
        for (size_t i = 0; i < (size_t)seq * D; ++i) x[i] = x[i] + y[i];
    }
    for (int i = 0; i < seq; ++i) rms_norm(x + (size_t)i * D, D, fnorm, c->eps, out + (size_t)i * D);
    rc = 0;
done:
    free(x); free(h); free(q); free(k); free(v); free(vt); free(o); free(y); free(f); free(bias); free(rowbuf);
    free(sc);
    return rc;
}

REF_API int ref_convention(void) { return 4; }

REF_API void ref_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}
REF_API int ref_get_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
