// kernels.hip -- gfx950 kernels for one MusicGen LM decode step.
//
// Every reduction runs in a fixed order that does not depend on the launch shape, and every
// floating-point step is spelled out (built with -ffp-contract=off), so a step is
// deterministic and reproduces the documented ggml-CPU conventions bit for bit:
//
//   * quantized GEMV: activation -> Q8_0 per 32-block (d = amax/127, q = roundf(x/d)),
//     exact integer block dots (v_dot4), term = (float)isum * (dw*dx), terms of a row summed
//     as 64 lane-strided partials (lane l owns blocks l, l+64, ...) then a xor butterfly;
//   * F16 / F32 GEMV: the same with 8-element chunks and fmaf;
//   * LayerNorm: double partial sums per lane, butterfly, (x-mean)*(1/sqrtf(var+eps))*w+b;
//   * attention: keys in chunks of 256; q.k as 16 four-dim fmaf partials + butterfly;
//     softmax sum in double per chunk (butterfly), chunks added in order; V as 16 key-strided
//     partials per chunk + butterfly, chunk results added in order;
//   * exp / erf: this file's own double routines (Cody-Waite + Taylor; Taylor / continued
//     fraction), rounded to f32 once.
//
// The reference computes the same steps through ggml (src/mg/lm.h:152-259, src/nn.h:186-191,
// src/ac/transformer.h:28-38, src/mg/sampling.h:32-105).
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "kernels.h"

namespace mgx {

// ------------------------------------------------------------------------------------
// scalar helpers
// ------------------------------------------------------------------------------------
__device__ __forceinline__ float h2f(uint16_t h) { return __half2float(__ushort_as_half(h)); }
__device__ __forceinline__ uint16_t f2h(float f) { return __half_as_ushort(__float2half_rn(f)); }

__device__ __constant__ double RECIP_FACT[14] = {
    1.0, 1.0, 0.5, 0.16666666666666666, 0.041666666666666664, 0.008333333333333333,
    0.001388888888888889, 0.0001984126984126984, 2.48015873015873e-05,
    2.7557319223985893e-06, 2.755731922398589e-07, 2.505210838544172e-08,
    2.08767569878681e-09, 1.6059043836821613e-10};

// e^x: x = k ln2 + r with ln2 split in two doubles, e^r by its Taylor series to r^13.
__device__ double dexp(double x) {
    if (x != x) return x;
    if (x > 709.782712893384) return __builtin_inf();
    if (x < -745.2) return 0.0;
    const double k = __builtin_rint(x * 1.4426950408889634);
    double r = __builtin_fma(-k, 0.6931471805599453, x);
    r = __builtin_fma(-k, 2.3190468138462996e-17, r);
    double p = 1.6059043836821613e-10;
    p = __builtin_fma(p, r, 2.08767569878681e-09);
    p = __builtin_fma(p, r, 2.505210838544172e-08);
    p = __builtin_fma(p, r, 2.755731922398589e-07);
    p = __builtin_fma(p, r, 2.7557319223985893e-06);
    p = __builtin_fma(p, r, 2.48015873015873e-05);
    p = __builtin_fma(p, r, 0.0001984126984126984);
    p = __builtin_fma(p, r, 0.001388888888888889);
    p = __builtin_fma(p, r, 0.008333333333333333);
    p = __builtin_fma(p, r, 0.041666666666666664);
    p = __builtin_fma(p, r, 0.16666666666666666);
    p = __builtin_fma(p, r, 0.5);
    p = __builtin_fma(p, r, 1.0);
    p = __builtin_fma(p, r, 1.0);
    return __builtin_ldexp(p, (int)k);
}
__device__ __forceinline__ float dexpf(float x) { return (float)dexp((double)x); }

__device__ __constant__ double ERF_TAYLOR[30] = {
    1.0, -0.3333333333333333, 0.1, -0.023809523809523808,
    0.004629629629629629, -0.0007575757575757576, 0.00010683760683760684, -1.3227513227513228e-05,
    1.4589169000933706e-06, -1.4503852223150468e-07, 1.3122532963802806e-08, -1.0892221037148573e-09,
    8.35070279514724e-11, -5.9477940136376354e-12, 3.9554295164585257e-13, -2.466827010264457e-14,
    1.4483264643598138e-15, -8.032735012415773e-17, 4.221407288807088e-18, -2.107855191442136e-19,
    1.0025164934907719e-20, -4.5518467589282e-22, 1.977064753877905e-23, -8.230149299214221e-25,
    3.289260349175752e-26, -1.2641078988989164e-27, 4.6784835155184856e-29, -1.669761793417372e-30,
    5.754191643982172e-32, -1.9169428621097826e-33};

// erf: Taylor series below |x| = 2, the Laplace continued fraction for erfc (forward
// three-term recurrence, 50 terms) up to 6, +-1 beyond.
__device__ double derf(double x) {
    const double ax = __builtin_fabs(x);
    if (ax < 2.0) {
        const double t = x * x;
        double p = ERF_TAYLOR[29];
        for (int n = 28; n >= 0; --n) p = __builtin_fma(p, t, ERF_TAYLOR[n]);
        return (x * p) * 1.1283791670955126;
    }
    if (ax >= 6.0) return x > 0 ? 1.0 : -1.0;
    double am2 = 1.0, am1 = 0.0, bm2 = 0.0, bm1 = 1.0;
    for (int n = 1; n <= 50; ++n) {
        const double a = (n == 1) ? 1.0 : 0.5 * (double)(n - 1);
        const double A = __builtin_fma(ax, am1, a * am2);
        const double B = __builtin_fma(ax, bm1, a * bm2);
        am2 = am1; am1 = A; bm2 = bm1; bm1 = B;
    }
    const double erfc = (dexp(-(ax * ax)) * 0.5641895835477563) * (am1 / bm1);
    const double r = 1.0 - erfc;
    return x > 0 ? r : -r;
}

// ggml_gelu_erf: 0.5*x*(1+erf(x/sqrt 2)) in f32 (lm.h:203).
__device__ __forceinline__ float gelu_erf(float x) {
    const float e = (float)derf((double)(x * 0.70710678118654752440f));
    return 0.5f * x * (1.0f + e);
}

template <typename T> __device__ __forceinline__ T shfl_xor(T v, int m) { return __shfl_xor(v, m, 64); }

// Butterfly over the 64 lanes of a wave: lane l < off adds lane l+off, off = 32..1.
__device__ __forceinline__ float fold64(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = v + shfl_xor(v, off);
    return v;
}
__device__ __forceinline__ double fold64d(double v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = v + shfl_xor(v, off);
    return v;
}

// Q8_0 activation quantization of one element per lane; lanes 32k..32k+31 form one block.
// Writes q and (from the block's first lane) the fp16-rounded scale widened to f32.
__device__ __forceinline__ void quant_q8_lane(float v, int lane, int8_t* qdst, float* ddst) {
    float amax = __builtin_fabsf(v);
#pragma unroll
    for (int off = 16; off >= 1; off >>= 1) {
        const float o = shfl_xor(amax, off);
        amax = amax > o ? amax : o;
    }
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    *qdst = (int8_t)__builtin_roundf(v * id);
    if ((lane & 31) == 0) *ddst = h2f(f2h(d));
}

// Writes element i (of a column) in the activation form the consumer's weights want.
__device__ __forceinline__ void put_act(const ActBuf& a, int col, int i, float v, int lane) {
    if (a.kind == ACT_Q8) quant_q8_lane(v, lane, a.q + (size_t)col * a.stride + i, a.d + (size_t)col * (a.stride / 32) + i / 32);
    else if (a.kind == ACT_F16) a.h[(size_t)col * a.stride + i] = f2h(v);
    else a.f[(size_t)col * a.stride + i] = v;
}

// ------------------------------------------------------------------------------------
// embedding: sum of n_q rows + sinusoid, broadcast to every stream (lm.h:231-240)
// ------------------------------------------------------------------------------------
__device__ __forceinline__ float mat_elem(const DevMat& m, int r, int i) {
    switch (m.type) {
    case T_Q8_0: return (float)((const int8_t*)m.q)[(size_t)r * m.in + i] * h2f(m.d[(size_t)r * (m.in / 32) + i / 32]);
    case T_Q4_0: {
        const uint8_t* blk = (const uint8_t*)m.q + (size_t)r * (m.in / 2) + (i / 32) * 16;
        const int j = i & 31;
        const int nib = j < 16 ? (blk[j] & 15) : (blk[j - 16] >> 4);
        return (float)(nib - 8) * h2f(m.d[(size_t)r * (m.in / 32) + i / 32]);
    }
    case T_F16: return h2f(((const uint16_t*)m.q)[(size_t)r * m.in + i]);
    default: return ((const float*)m.q)[(size_t)r * m.in + i];
    }
}

__global__ __launch_bounds__(256) void k_embed(EmbedArgs a) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= a.dim) return;
    float e = 0.0f;
    for (int q = 0; q < a.n_q; ++q) {
        const int id = a.ids[(size_t)q * a.ids_stride];
        const float v = mat_elem(a.emb[q], id, i);
        e = q == 0 ? v : e + v;
    }
    const float x = a.pos[(size_t)a.position * a.dim + i] + e;
    for (int n = 0; n < a.ncol; ++n) a.x[(size_t)n * a.dim + i] = x;
}

// ------------------------------------------------------------------------------------
// LayerNorm of one column per wave, then conversion to the activation form
// (transformer.h:28-38; the ggml_norm arithmetic is spelled out in the file header)
// ------------------------------------------------------------------------------------
__global__ __launch_bounds__(64) void k_ln_act(LnArgs a) {
    const int col = blockIdx.x, lane = threadIdx.x;
    const float* x = a.x + (size_t)col * a.x_stride;
    const int n = a.dim;
    double s = 0.0;
    for (int i = lane; i < n; i += 64) s = s + (double)x[i];
    s = fold64d(s);
    const float mean = (float)(s / (double)n);
    double s2 = 0.0;
    for (int i = lane; i < n; i += 64) {
        const float v = x[i] - mean;
        s2 = s2 + (double)(v * v);
    }
    s2 = fold64d(s2);
    const float var = (float)(s2 / (double)n);
    const float scale = 1.0f / __builtin_sqrtf(var + a.eps);
    for (int i = lane; i < n; i += 64) {
        float v = x[i] - mean;
        v = v * scale;
        v = v * a.w[i];
        v = v + a.b[i];
        put_act(a.out, col, i, v, lane);
    }
}

// f32 columns -> activation form (the GELU output before ff.2).
__global__ __launch_bounds__(256) void k_act(ActArgs a) {
    const int col = blockIdx.y;
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= a.n) return;
    put_act(a.out, col, i, a.x[(size_t)col * a.x_stride + i], threadIdx.x & 63);
}

__global__ __launch_bounds__(256) void k_add_bias(float* y, const float* b, int n, int ncol) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n * ncol) return;
    y[i] = y[i] + b[i % n];
}

// ------------------------------------------------------------------------------------
// GEMV: y[col][r] = W[r] . act[col], one wave per row, lane l owns blocks l, l+64, ...
// ------------------------------------------------------------------------------------
template <int NC>
__device__ __forceinline__ void gemv_epilogue(const GemvArgs& a, int r, const float* acc, int ncol) {
    const GemvOut& o = a.o;
    for (int n = 0; n < ncol && n < NC; ++n) {
        const float v = acc[n];
        switch (o.mode) {
        case EPI_STORE: o.y[(size_t)n * o.y_stride + r] = v; break;
        case EPI_RESID: { float* p = o.y + (size_t)n * o.y_stride + r; *p = *p + v; break; }
        case EPI_GELU: o.y[(size_t)n * o.y_stride + r] = gelu_erf(v); break;
        case EPI_QKV: {
            const int sec = r / o.dim, w = r - sec * o.dim, head = w >> 6, dim = w & 63;
            if (sec == 0) o.y[(size_t)n * o.dim + w] = v;
            else {
                float* cache = sec == 1 ? o.k : o.v;
                cache[(((size_t)n * o.heads + head) * o.cap + o.position) * 64 + dim] = v;
            }
            break;
        }
        }
    }
}

template <int NC>
__global__ __launch_bounds__(256) void k_gemv_q8(GemvArgs a) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + wave;
    if (r >= a.w.out) return;
    const int in = a.w.in, nb = in / 32;
    const int8_t* wq = (const int8_t*)a.w.q + (size_t)r * in;
    const uint16_t* wd = a.w.d + (size_t)r * nb;
    float part[NC];
#pragma unroll
    for (int n = 0; n < NC; ++n) part[n] = 0.0f;
    for (int b = lane; b < nb; b += 64) {
        const int4 w0 = *(const int4*)(wq + b * 32), w1 = *(const int4*)(wq + b * 32 + 16);
        const float dw = h2f(wd[b]);
#pragma unroll
        for (int n = 0; n < NC; ++n) {
            if (n >= a.ncol) break;
            const int8_t* xq = a.act.q + (size_t)n * a.act.stride + b * 32;
            const int4 x0 = *(const int4*)xq, x1 = *(const int4*)(xq + 16);
            int s = __builtin_amdgcn_sdot4(w0.x, x0.x, 0, false);
            s = __builtin_amdgcn_sdot4(w0.y, x0.y, s, false);
            s = __builtin_amdgcn_sdot4(w0.z, x0.z, s, false);
            s = __builtin_amdgcn_sdot4(w0.w, x0.w, s, false);
            s = __builtin_amdgcn_sdot4(w1.x, x1.x, s, false);
            s = __builtin_amdgcn_sdot4(w1.y, x1.y, s, false);
            s = __builtin_amdgcn_sdot4(w1.z, x1.z, s, false);
            s = __builtin_amdgcn_sdot4(w1.w, x1.w, s, false);
            const float dd = dw * a.act.d[(size_t)n * (a.act.stride / 32) + b];
            const float term = (float)s * dd;
            part[n] = part[n] + term;
        }
    }
#pragma unroll
    for (int n = 0; n < NC; ++n) part[n] = fold64(part[n]);
    if (lane == 0) gemv_epilogue<NC>(a, r, part, a.ncol);
}

// Q4_0: sum((nib-8)*x) = sum(nib*x) - 8*sum(x), both exact integer dots.
__device__ __forceinline__ int q4_isum(const int4 w, const int4 x0, const int4 x1) {
    const uint32_t ws[4] = {(uint32_t)w.x, (uint32_t)w.y, (uint32_t)w.z, (uint32_t)w.w};
    const int xl[4] = {x0.x, x0.y, x0.z, x0.w}, xh[4] = {x1.x, x1.y, x1.z, x1.w};
    int s = 0, sx = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        s = __builtin_amdgcn_sdot4((int)(ws[k] & 0x0f0f0f0fu), xl[k], s, false);
        s = __builtin_amdgcn_sdot4((int)((ws[k] >> 4) & 0x0f0f0f0fu), xh[k], s, false);
        sx = __builtin_amdgcn_sdot4(0x01010101, xl[k], sx, false);
        sx = __builtin_amdgcn_sdot4(0x01010101, xh[k], sx, false);
    }
    return s - 8 * sx;
}

template <int NC>
__global__ __launch_bounds__(256) void k_gemv_q4(GemvArgs a) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + wave;
    if (r >= a.w.out) return;
    const int in = a.w.in, nb = in / 32;
    const uint8_t* wq = (const uint8_t*)a.w.q + (size_t)r * (in / 2);
    const uint16_t* wd = a.w.d + (size_t)r * nb;
    float part[NC];
#pragma unroll
    for (int n = 0; n < NC; ++n) part[n] = 0.0f;
    for (int b = lane; b < nb; b += 64) {
        const int4 w = *(const int4*)(wq + b * 16);
        const float dw = h2f(wd[b]);
#pragma unroll
        for (int n = 0; n < NC; ++n) {
            if (n >= a.ncol) break;
            const int8_t* xq = a.act.q + (size_t)n * a.act.stride + b * 32;
            const int s = q4_isum(w, *(const int4*)xq, *(const int4*)(xq + 16));
            const float dd = dw * a.act.d[(size_t)n * (a.act.stride / 32) + b];
            const float term = (float)s * dd;
            part[n] = part[n] + term;
        }
    }
#pragma unroll
    for (int n = 0; n < NC; ++n) part[n] = fold64(part[n]);
    if (lane == 0) gemv_epilogue<NC>(a, r, part, a.ncol);
}

// F16 weights x fp16-rounded activations (products exact in f32), 8-element chunks.
template <int NC>
__global__ __launch_bounds__(256) void k_gemv_f16(GemvArgs a) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + wave;
    if (r >= a.w.out) return;
    const int in = a.w.in, nch = in / 8;
    const uint16_t* w = (const uint16_t*)a.w.q + (size_t)r * in;
    float part[NC];
#pragma unroll
    for (int n = 0; n < NC; ++n) part[n] = 0.0f;
    for (int c = lane; c < nch; c += 64) {
        const int4 wv = *(const int4*)(w + c * 8);
        const uint16_t* wh = (const uint16_t*)&wv;
#pragma unroll
        for (int n = 0; n < NC; ++n) {
            if (n >= a.ncol) break;
            const int4 xv = *(const int4*)(a.act.h + (size_t)n * a.act.stride + c * 8);
            const uint16_t* xh = (const uint16_t*)&xv;
            float p = part[n];
#pragma unroll
            for (int e = 0; e < 8; ++e) p = __builtin_fmaf(h2f(wh[e]), h2f(xh[e]), p);
            part[n] = p;
        }
    }
#pragma unroll
    for (int n = 0; n < NC; ++n) part[n] = fold64(part[n]);
    if (lane == 0) gemv_epilogue<NC>(a, r, part, a.ncol);
}

template <int NC>
__global__ __launch_bounds__(256) void k_gemv_f32(GemvArgs a) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + wave;
    if (r >= a.w.out) return;
    const int in = a.w.in, nch = in / 8;
    const float* w = (const float*)a.w.q + (size_t)r * in;
    float part[NC];
#pragma unroll
    for (int n = 0; n < NC; ++n) part[n] = 0.0f;
    for (int c = lane; c < nch; c += 64) {
        const float4 w0 = *(const float4*)(w + c * 8), w1 = *(const float4*)(w + c * 8 + 4);
        const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
        for (int n = 0; n < NC; ++n) {
            if (n >= a.ncol) break;
            const float* x = a.act.f + (size_t)n * a.act.stride + c * 8;
            float p = part[n];
#pragma unroll
            for (int e = 0; e < 8; ++e) p = __builtin_fmaf(wv[e], x[e], p);
            part[n] = p;
        }
    }
#pragma unroll
    for (int n = 0; n < NC; ++n) part[n] = fold64(part[n]);
    if (lane == 0) gemv_epilogue<NC>(a, r, part, a.ncol);
}

// ------------------------------------------------------------------------------------
// decode self-attention over keys [0, position] (nn.h:186-191, no mask for one query)
// ------------------------------------------------------------------------------------
// Scores of one 256-key chunk: 16 lanes per key, each lane four dims.
__global__ __launch_bounds__(256) void k_attn_scores(AttnArgs a) {
    const int c = blockIdx.x, h = blockIdx.y, n = blockIdx.z;
    const int u = a.position + 1;
    if (c * ATT_CHUNK >= u) return;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, t = lane & 15;
    const size_t head = (size_t)n * a.heads + h;
    const float* K = a.k + head * a.cap * 64;
    const float4 q = ((const float4*)(a.q + (size_t)n * a.dim + h * 64))[t];
    float* S = a.scores + head * a.cap;
    for (int it = 0; it < ATT_CHUNK / 16; ++it) {
        const int j = c * ATT_CHUNK + it * 16 + wave * 4 + g;
        float p = 0.0f;
        if (j < u) {
            const float4 k = ((const float4*)(K + (size_t)j * 64))[t];
            p = __builtin_fmaf(q.x, k.x, 0.0f);
            p = __builtin_fmaf(q.y, k.y, p);
            p = __builtin_fmaf(q.z, k.z, p);
            p = __builtin_fmaf(q.w, k.w, p);
        }
        p = p + shfl_xor(p, 8);
        p = p + shfl_xor(p, 4);
        p = p + shfl_xor(p, 2);
        p = p + shfl_xor(p, 1);
        if (t == 0 && j < u) S[j] = p * a.scale;
    }
}

// Max and softmax denominator over all keys (redone by every chunk's block, deterministic),
// then this chunk's share of V^T p.
__global__ __launch_bounds__(256) void k_attn_softmax_v(AttnArgs a) {
    const int c = blockIdx.x, h = blockIdx.y, n = blockIdx.z;
    const int u = a.position + 1;
    if (c * ATT_CHUNK >= u) return;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const size_t head = (size_t)n * a.heads + h;
    const float* S = a.scores + head * a.cap;
    __shared__ float red_f[4];
    __shared__ double red_d[256];
    __shared__ float pv[ATT_CHUNK];
    __shared__ float4 vred[16][16];
    __shared__ float inv_sh;
    float mx = -__builtin_inff();
    for (int j = tid; j < u; j += 256) { const float s = S[j]; mx = mx > s ? mx : s; }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) { const float o = shfl_xor(mx, off); mx = mx > o ? mx : o; }
    if (lane == 0) red_f[wave] = mx;
    __syncthreads();
    mx = red_f[0];
    for (int w = 1; w < 4; ++w) mx = mx > red_f[w] ? mx : red_f[w];
    const int nch = (u + ATT_CHUNK - 1) / ATT_CHUNK;
    double total = 0.0;
    for (int cc = 0; cc < nch; ++cc) {
        const int j = cc * ATT_CHUNK + tid;
        red_d[tid] = j < u ? (double)dexpf(S[j] - mx) : 0.0;
        __syncthreads();
        if (tid < 128) red_d[tid] = red_d[tid] + red_d[tid + 128];
        __syncthreads();
        if (tid < 64) {
            double v = red_d[tid] + red_d[tid + 64];
            v = fold64d(v);
            if (tid == 0) total = total + v;
        }
        __syncthreads();
    }
    if (tid == 0) inv_sh = (float)(1.0 / total);
    __syncthreads();
    const float inv = inv_sh;
    {
        const int j = c * ATT_CHUNK + tid;
        pv[tid] = j < u ? dexpf(S[j] - mx) * inv : 0.0f;
    }
    __syncthreads();
    // V pass: partial g = key mod 16 (g = 4*wave + lane/16), lane%16 -> dims 4*(lane%16)..+3.
    const int g = wave * 4 + (lane >> 4), dq = lane & 15;
    const float* V = a.v + head * a.cap * 64;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int m = 0; m < ATT_CHUNK / 16; ++m) {
        const int jj = g + 16 * m, j = c * ATT_CHUNK + jj;
        if (j < u) {
            const float p = pv[jj];
            const float4 v = ((const float4*)(V + (size_t)j * 64))[dq];
            acc.x = __builtin_fmaf(p, v.x, acc.x);
            acc.y = __builtin_fmaf(p, v.y, acc.y);
            acc.z = __builtin_fmaf(p, v.z, acc.z);
            acc.w = __builtin_fmaf(p, v.w, acc.w);
        }
    }
    vred[g][dq] = acc;
    __syncthreads();
    if (g < 8) {
        const float4 o = vred[g + 8][dq];
        vred[g][dq] = make_float4(acc.x + o.x, acc.y + o.y, acc.z + o.z, acc.w + o.w);
    }
    __syncthreads();
    if (g < 4) {
        const float4 s = vred[g][dq], o = vred[g + 4][dq];
        float4 r = make_float4(s.x + o.x, s.y + o.y, s.z + o.z, s.w + o.w);
        // g = lane>>4 in wave 0: off 2 -> lane xor 32, off 1 -> lane xor 16
        r.x = r.x + shfl_xor(r.x, 32); r.y = r.y + shfl_xor(r.y, 32);
        r.z = r.z + shfl_xor(r.z, 32); r.w = r.w + shfl_xor(r.w, 32);
        r.x = r.x + shfl_xor(r.x, 16); r.y = r.y + shfl_xor(r.y, 16);
        r.z = r.z + shfl_xor(r.z, 16); r.w = r.w + shfl_xor(r.w, 16);
        if (g == 0) ((float4*)(a.opart + (head * a.max_chunks + c) * 64))[dq] = r;
    }
}

// Chunk results added in order, then the head's 64 outputs go to the out-proj activation.
__global__ __launch_bounds__(64) void k_attn_reduce(AttnArgs a, ActBuf out) {
    const int h = blockIdx.x, n = blockIdx.y, lane = threadIdx.x;
    const int u = a.position + 1, nch = (u + ATT_CHUNK - 1) / ATT_CHUNK;
    const size_t head = (size_t)n * a.heads + h;
    float r = 0.0f;
    for (int c = 0; c < nch; ++c) r = r + a.opart[(head * a.max_chunks + c) * 64 + lane];
    put_act(out, n, h * 64 + lane, r, lane);
}

// ------------------------------------------------------------------------------------
// cross-attention of the conditional stream over the projected memory (lm.h:181-199).
// The null stream's memory is zero, so its block output is exactly zero and is skipped.
// ------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_xattn(XAttnArgs a) {
    const int h = blockIdx.x;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, t = lane & 15;
    const int nc = a.n_ctx;
    const float* K = a.k + (size_t)h * nc * 64;
    const float* V = a.v + (size_t)h * nc * 64;
    __shared__ float s[256];
    __shared__ float red_f[4];
    __shared__ double red_d[256];
    __shared__ float4 vred[16][16];
    __shared__ float inv_sh;
    const float4 q = ((const float4*)(a.q + h * 64))[t];
    for (int it = 0; it * 16 < nc; ++it) {
        const int j = it * 16 + wave * 4 + g;
        float p = 0.0f;
        if (j < nc) {
            const float4 k = ((const float4*)(K + (size_t)j * 64))[t];
            p = __builtin_fmaf(q.x, k.x, 0.0f);
            p = __builtin_fmaf(q.y, k.y, p);
            p = __builtin_fmaf(q.z, k.z, p);
            p = __builtin_fmaf(q.w, k.w, p);
        }
        p = p + shfl_xor(p, 8);
        p = p + shfl_xor(p, 4);
        p = p + shfl_xor(p, 2);
        p = p + shfl_xor(p, 1);
        if (t == 0 && j < nc) s[j] = p * a.scale;
    }
    __syncthreads();
    float mx = -__builtin_inff();
    for (int j = tid; j < nc; j += 256) mx = mx > s[j] ? mx : s[j];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) { const float o = shfl_xor(mx, off); mx = mx > o ? mx : o; }
    if (lane == 0) red_f[wave] = mx;
    __syncthreads();
    mx = red_f[0];
    for (int w = 1; w < 4; ++w) mx = mx > red_f[w] ? mx : red_f[w];
    const float e = tid < nc ? dexpf(s[tid] - mx) : 0.0f;
    red_d[tid] = tid < nc ? (double)e : 0.0;
    __syncthreads();
    if (tid < 128) red_d[tid] = red_d[tid] + red_d[tid + 128];
    __syncthreads();
    if (tid < 64) {
        double v = red_d[tid] + red_d[tid + 64];
        v = fold64d(v);
        if (tid == 0) inv_sh = (float)(1.0 / (0.0 + v));
    }
    __syncthreads();
    if (tid < nc) s[tid] = e * inv_sh;
    __syncthreads();
    const int gg = wave * 4 + g, dq = lane & 15;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int m = 0; gg + 16 * m < nc; ++m) {
        const int j = gg + 16 * m;
        const float p = s[j];
        const float4 v = ((const float4*)(V + (size_t)j * 64))[dq];
        acc.x = __builtin_fmaf(p, v.x, acc.x);
        acc.y = __builtin_fmaf(p, v.y, acc.y);
        acc.z = __builtin_fmaf(p, v.z, acc.z);
        acc.w = __builtin_fmaf(p, v.w, acc.w);
    }
    vred[gg][dq] = acc;
    __syncthreads();
    if (gg < 8) {
        const float4 o = vred[gg + 8][dq];
        vred[gg][dq] = make_float4(acc.x + o.x, acc.y + o.y, acc.z + o.z, acc.w + o.w);
    }
    __syncthreads();
    if (gg < 4) {
        const float4 sv = vred[gg][dq], o = vred[gg + 4][dq];
        float4 r = make_float4(sv.x + o.x, sv.y + o.y, sv.z + o.z, sv.w + o.w);
        r.x = r.x + shfl_xor(r.x, 32); r.y = r.y + shfl_xor(r.y, 32);
        r.z = r.z + shfl_xor(r.z, 32); r.w = r.w + shfl_xor(r.w, 32);
        r.x = r.x + shfl_xor(r.x, 16); r.y = r.y + shfl_xor(r.y, 16);
        r.z = r.z + shfl_xor(r.z, 16); r.w = r.w + shfl_xor(r.w, 16);
        if (gg == 0) ((float4*)a.o)[h * 16 + dq] = make_float4(0.0f + r.x, 0.0f + r.y, 0.0f + r.z, 0.0f + r.w);
    }
}

// The hoisted cross K/V: projected [n_ctx][2*dim] -> K [H][n_ctx][64], V [H][n_ctx][64].
__global__ __launch_bounds__(256) void k_xkv_split(const float* kv, int n_ctx, int dim, float* k, float* v) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n_ctx * 2 * dim) return;
    const int t = i / (2 * dim), r = i - t * 2 * dim;
    const int sec = r / dim, w = r - sec * dim, head = w >> 6, d = w & 63;
    (sec == 0 ? k : v)[((size_t)head * n_ctx + t) * 64 + d] = kv[i];
}

// ------------------------------------------------------------------------------------
// sampling: CFG mix + argmax / softmax, top-k, categorical (pipeline.cpp:264-294,
// sampling.h:32-105), one block per codebook
// ------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_sample(SampleArgs a) {
    const int q = blockIdx.x, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int C = a.card;
    __shared__ float lg[MAX_CARD];
    __shared__ double ex[MAX_CARD];
    __shared__ float pr[MAX_CARD];
    __shared__ uint32_t hist[256];
    __shared__ float red_f[4];
    __shared__ int red_i[4];
    __shared__ int tok_sh;
    __shared__ float inv_sh;
    __shared__ uint32_t prefix_sh;
    __shared__ int k_sh;
    const float* cond = a.logits + (size_t)q * C;
    const float* null_l = a.logits + (size_t)(a.n_q + q) * C;
    for (int i = tid; i < C; i += 256) {
        float v = cond[i];
        if (a.guided) v = null_l[i] + (cond[i] - null_l[i]) * a.cfg_coef;
        lg[i] = v;
        if (a.first_logits) a.first_logits[(size_t)q * C + i] = v;
        if (a.step_logits) a.step_logits[(size_t)q * C + i] = v;
    }
    __syncthreads();
    const int offset = a.offset;
    const bool live = a.mask[(size_t)q * a.steps + offset] != 0;
    int token;
    if (!live) token = a.special;
    else if (!a.use_sampling || !(a.temperature > 0.0f)) {
        // argmax, lowest index on ties
        float best = -__builtin_inff();
        int bi = 0x7fffffff;
        for (int i = tid; i < C; i += 256)
            if (lg[i] > best || (lg[i] == best && i < bi)) { best = lg[i]; bi = i; }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            const float ob = shfl_xor(best, off);
            const int oi = shfl_xor(bi, off);
            if (ob > best || (ob == best && oi < bi)) { best = ob; bi = oi; }
        }
        if (lane == 0) { red_f[wave] = best; red_i[wave] = bi; }
        __syncthreads();
        if (tid == 0) {
            float b = red_f[0]; int ii = red_i[0];
            for (int w = 1; w < 4; ++w)
                if (red_f[w] > b || (red_f[w] == b && red_i[w] < ii)) { b = red_f[w]; ii = red_i[w]; }
            tok_sh = ii;
        }
        __syncthreads();
        token = tok_sh;
    } else {
        // softmax_into: peak, double exps, sequential double total, float scale
        float pk = -__builtin_inff();
        for (int i = tid; i < C; i += 256) pk = pk < lg[i] ? lg[i] : pk;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) { const float o = shfl_xor(pk, off); pk = pk < o ? o : pk; }
        if (lane == 0) red_f[wave] = pk;
        __syncthreads();
        pk = red_f[0];
        for (int w = 1; w < 4; ++w) pk = pk < red_f[w] ? red_f[w] : pk;
        for (int i = tid; i < C; i += 256) {
            const double e = dexp(((double)lg[i] - (double)pk) / (double)a.temperature);
            ex[i] = e;
            pr[i] = (float)e;
        }
        __syncthreads();
        if (tid == 0) {
            double total = 0.0;
            for (int i = 0; i < C; ++i) total += ex[i];
            inv_sh = (float)(1.0 / total);
        }
        __syncthreads();
        for (int i = tid; i < C; i += 256) pr[i] = pr[i] * inv_sh;
        __syncthreads();
        // top_k_filter: the k-th largest value (counting repeats) by MSB-first radix select
        // over the bit patterns (non-negative floats order like their bits).
        const int k = a.top_k;
        if (k > 0 && k < C) {
            if (tid == 0) { prefix_sh = 0; k_sh = k; }
            __syncthreads();
            for (int shift = 24; shift >= 0; shift -= 8) {
                hist[tid] = 0;
                __syncthreads();
                const uint32_t pre = prefix_sh;
                const uint32_t hmask = shift == 24 ? 0u : (0xffffffffu << (shift + 8));
                for (int i = tid; i < C; i += 256) {
                    const uint32_t bits = __float_as_uint(pr[i]);
                    if ((bits & hmask) == (pre & hmask)) atomicAdd(&hist[(bits >> shift) & 255u], 1u);
                }
                __syncthreads();
                if (tid == 0) {
                    int kk = k_sh;
                    int bin = 255;
                    for (; bin > 0; --bin) {
                        if ((int)hist[bin] >= kk) break;
                        kk -= (int)hist[bin];
                    }
                    k_sh = kk;
                    prefix_sh = pre | ((uint32_t)bin << shift);
                }
                __syncthreads();
            }
            const float cutoff = __uint_as_float(prefix_sh);
            for (int i = tid; i < C; i += 256) if (pr[i] < cutoff) pr[i] = 0.0f;
            __syncthreads();
            if (tid == 0) {
                double total = 0.0;
                for (int i = 0; i < C; ++i) total += (double)pr[i];
                inv_sh = (float)(1.0 / total);
            }
            __syncthreads();
            for (int i = tid; i < C; i += 256) pr[i] = pr[i] * inv_sh;
            __syncthreads();
        }
        // categorical(probs, 1.0): first i whose running double sum exceeds u
        if (tid == 0) {
            const double target = (double)a.uniforms[(size_t)offset * a.n_q + q] * 1.0;
            double acc = 0.0;
            int pick = C - 1;
            for (int i = 0; i < C; ++i) {
                acc += (double)pr[i];
                if (acc > target) { pick = i; break; }
            }
            tok_sh = pick;
        }
        __syncthreads();
        token = tok_sh;
    }
    if (tid == 0) {
        int32_t* slot = a.seq + (size_t)q * a.steps + offset;
        if (*slot == -1) *slot = token;
    }
}

// ------------------------------------------------------------------------------------
// launchers
// ------------------------------------------------------------------------------------
void launch_embed(const EmbedArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(k_embed, dim3((a.dim + 255) / 256), dim3(256), 0, s, a);
}
void launch_ln_act(const LnArgs& a, int ncol, hipStream_t s) {
    hipLaunchKernelGGL(k_ln_act, dim3(ncol), dim3(64), 0, s, a);
}
void launch_act(const ActArgs& a, int ncol, hipStream_t s) {
    hipLaunchKernelGGL(k_act, dim3((a.n + 255) / 256, ncol), dim3(256), 0, s, a);
}
void launch_add_bias(float* y, const float* b, int n, int ncol, hipStream_t s) {
    hipLaunchKernelGGL(k_add_bias, dim3((n * ncol + 255) / 256), dim3(256), 0, s, y, b, n, ncol);
}

template <int NC> static void gemv_nc(const GemvArgs& a, hipStream_t s) {
    const dim3 grid((a.w.out + 3) / 4), block(256);
    switch (a.w.type) {
    case T_Q8_0: hipLaunchKernelGGL(k_gemv_q8<NC>, grid, block, 0, s, a); break;
    case T_Q4_0: hipLaunchKernelGGL(k_gemv_q4<NC>, grid, block, 0, s, a); break;
    case T_F16: hipLaunchKernelGGL(k_gemv_f16<NC>, grid, block, 0, s, a); break;
    default: hipLaunchKernelGGL(k_gemv_f32<NC>, grid, block, 0, s, a); break;
    }
}
void launch_gemv(const GemvArgs& a, hipStream_t s) {
    if (a.ncol <= 1) gemv_nc<1>(a, s);
    else if (a.ncol <= 2) gemv_nc<2>(a, s);
    else if (a.ncol <= 4) gemv_nc<4>(a, s);
    else if (a.ncol <= 8) gemv_nc<8>(a, s);
    else gemv_nc<16>(a, s);
}
void launch_attention(const AttnArgs& a, const ActBuf& out, hipStream_t s) {
    const dim3 grid(a.max_chunks, a.heads, a.ncol);
    hipLaunchKernelGGL(k_attn_scores, grid, dim3(256), 0, s, a);
    hipLaunchKernelGGL(k_attn_softmax_v, grid, dim3(256), 0, s, a);
    hipLaunchKernelGGL(k_attn_reduce, dim3(a.heads, a.ncol), dim3(64), 0, s, a, out);
}
void launch_xattn(const XAttnArgs& a, int heads, hipStream_t s) {
    hipLaunchKernelGGL(k_xattn, dim3(heads), dim3(256), 0, s, a);
}
void launch_xkv_split(const float* kv, int n_ctx, int dim, float* k, float* v, hipStream_t s) {
    hipLaunchKernelGGL(k_xkv_split, dim3((n_ctx * 2 * dim + 255) / 256), dim3(256), 0, s, kv, n_ctx, dim, k, v);
}
void launch_sample(const SampleArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(k_sample, dim3(a.n_q), dim3(256), 0, s, a);
}

}  // namespace mgx

namespace mgx {

// ggml blocks -> device layout: Q8_0 {d, q[32]} rows split into q[out][in] + d[out][in/32];
// Q4_0 {d, qs[16]} into qs[out][in/2] + d. One thread per block.
__global__ __launch_bounds__(256) void k_repack(int type, const uint8_t* raw, int64_t nblocks, int8_t* q, uint16_t* d) {
    const int64_t b = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (b >= nblocks) return;
    if (type == T_Q8_0) {
        const uint8_t* src = raw + b * 34;
        d[b] = (uint16_t)(src[0] | (src[1] << 8));
        for (int j = 0; j < 32; ++j) q[b * 32 + j] = (int8_t)src[2 + j];
    } else {
        const uint8_t* src = raw + b * 18;
        d[b] = (uint16_t)(src[0] | (src[1] << 8));
        for (int j = 0; j < 16; ++j) q[b * 16 + j] = (int8_t)src[2 + j];
    }
}

void launch_repack(int type, const uint8_t* raw, int64_t rows, int in, void* q, uint16_t* d, hipStream_t s) {
    const int64_t nblocks = rows * (in / 32);
    hipLaunchKernelGGL(k_repack, dim3((unsigned)((nblocks + 255) / 256)), dim3(256), 0, s, type, raw, nblocks, (int8_t*)q, d);
}

}  // namespace mgx
