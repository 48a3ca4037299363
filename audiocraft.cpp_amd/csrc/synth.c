/*
 * synth.c -- seeded synthetic MusicGen-LM weights in ggml block formats.
 *
 * The benchmark and the parity tests need real-shaped models without checkpoints: every
 * 2-D matrix N(0, std), written straight into the GGUF tensor layout that the reference's
 * loader hands to ggml (gguf_model.h:363-414) -- F32, F16, Q8_0 {fp16 d; int8 q[32]} or
 * Q4_0 {fp16 d; uint8 qs[16]} with low nibbles holding elements 0..15 of a block and high
 * nibbles 16..31. Both the HIP library and the CPU oracle read the same bytes.
 *
 * Values are counter-based (splitmix64 of seed + index, Box-Muller in double), so any
 * subrange can be produced independently and in parallel, and a tensor's bytes depend only
 * on (seed, shape, type).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define API __attribute__((visibility("default")))

enum { T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q8_0 = 8 };

static inline uint64_t splitmix64(uint64_t z) {
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}
static inline double unit(uint64_t r) { return ((double)(r >> 11) + 1.0) * (1.0 / 9007199254740992.0); }

/* FNV-1a of a tensor name, mixed with a base seed: one independent stream per tensor. */
API uint64_t mgx_synth_seed(uint64_t base, const char* name) {
    uint64_t h = 1469598103934665603ull;
    for (const unsigned char* p = (const unsigned char*)name; *p; ++p) { h ^= *p; h *= 1099511628211ull; }
    return splitmix64(h ^ splitmix64(base));
}

/* Element i of a N(0, std) stream. */
static inline float normal_at(uint64_t seed, uint64_t i, float std) {
    const uint64_t k = i >> 1;
    const double u1 = unit(splitmix64(seed + 2 * k)), u2 = unit(splitmix64(seed + 2 * k + 1));
    const double r = sqrt(-2.0 * log(u1)), th = 6.283185307179586 * u2;
    return (float)((double)std * r * ((i & 1) ? sin(th) : cos(th)));
}

API void mgx_synth_normal(uint64_t seed, float std, float* out, uint64_t n) {
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)n; ++i) out[i] = normal_at(seed, (uint64_t)i, std);
}

/* Uniform integers in [0, hi). */
API void mgx_synth_codes(uint64_t seed, int32_t hi, int32_t* out, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) out[i] = (int32_t)(splitmix64(seed + i) % (uint64_t)hi);
}

static uint16_t f32_to_f16(float f) {
    uint32_t x; memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
    if (ax < 0x38800000u) {
        if (ax < 0x33000000u) return (uint16_t)sign;
        const int e = (int)(ax >> 23);
        const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        const int shift = 126 - e;
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

/* One row of n floats into `type` bytes (ggml quantize_row_*_ref conventions). */
static void pack_row(int type, const float* x, int n, uint8_t* out) {
    if (type == T_F32) { memcpy(out, x, sizeof(float) * (size_t)n); return; }
    if (type == T_F16) {
        for (int i = 0; i < n; ++i) { const uint16_t h = f32_to_f16(x[i]); memcpy(out + 2 * i, &h, 2); }
        return;
    }
    for (int b = 0; b < n / 32; ++b) {
        const float* v = x + 32 * b;
        if (type == T_Q8_0) {
            float amax = 0.0f;
            for (int j = 0; j < 32; ++j) { const float a = fabsf(v[j]); amax = amax > a ? amax : a; }
            const float d = amax / 127.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
            const uint16_t h = f32_to_f16(d);
            uint8_t* blk = out + 34 * b;
            memcpy(blk, &h, 2);
            for (int j = 0; j < 32; ++j) ((int8_t*)(blk + 2))[j] = (int8_t)roundf(v[j] * id);
        } else {
            float amax = 0.0f, mx = 0.0f;
            for (int j = 0; j < 32; ++j) {
                const float a = fabsf(v[j]);
                if (a > amax) { amax = a; mx = v[j]; }
            }
            const float d = mx / -8.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
            const uint16_t h = f32_to_f16(d);
            uint8_t* blk = out + 18 * b;
            memcpy(blk, &h, 2);
            for (int j = 0; j < 16; ++j) {
                int q0 = (int)(v[j] * id + 8.5f), q1 = (int)(v[j + 16] * id + 8.5f);
                q0 = q0 > 15 ? 15 : q0; q1 = q1 > 15 ? 15 : q1;
                blk[2 + j] = (uint8_t)(q0 | (q1 << 4));
            }
        }
    }
}

API uint64_t mgx_row_bytes(int type, int64_t ne0) {
    switch (type) {
    case T_F32: return (uint64_t)ne0 * 4;
    case T_F16: return (uint64_t)ne0 * 2;
    case T_Q8_0: return (uint64_t)(ne0 / 32) * 34;
    case T_Q4_0: return (uint64_t)(ne0 / 32) * 18;
    }
    return 0;
}

/* A [ne1 rows][ne0] N(0, std) matrix (or a constant when std == 0) in `type` bytes. */
API int mgx_synth_tensor(uint64_t seed, int type, int64_t ne0, int64_t ne1, float std, float constant, uint8_t* out) {
    if ((type == T_Q8_0 || type == T_Q4_0) && ne0 % 32) return -1;
    const uint64_t rb = mgx_row_bytes(type, ne0);
    if (!rb) return -1;
    #pragma omp parallel for schedule(dynamic, 16)
    for (int64_t r = 0; r < ne1; ++r) {
        float buf[8192];
        float* x = buf;
        float* heap = 0;
        if (ne0 > 8192) { heap = (float*)__builtin_malloc(sizeof(float) * (size_t)ne0); x = heap; }
        for (int64_t i = 0; i < ne0; ++i)
            x[i] = std != 0.0f ? normal_at(seed, (uint64_t)(r * ne0 + i), std) : constant;
        pack_row(type, x, (int)ne0, out + (uint64_t)r * rb);
        if (heap) __builtin_free(heap);
    }
    return 0;
}

/* Packs caller floats (e.g. a test's own values) into `type` bytes. */
API int mgx_pack(int type, const float* x, int64_t ne0, int64_t ne1, uint8_t* out) {
    if ((type == T_Q8_0 || type == T_Q4_0) && ne0 % 32) return -1;
    const uint64_t rb = mgx_row_bytes(type, ne0);
    for (int64_t r = 0; r < ne1; ++r) pack_row(type, x + r * ne0, (int)ne0, out + (uint64_t)r * rb);
    return 0;
}
