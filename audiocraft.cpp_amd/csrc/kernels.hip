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
//   * LayerNorm: 256 double partials (partial i sums float4 groups i, i+256, ... in element
//     order), butterfly, (x-mean)*(1/sqrtf(var+eps))*w+b;
//   * attention: keys in chunks of 256; q.k as 16 four-dim fmaf partials + butterfly; per
//     chunk its max m, e = expf(s - m), the sum of e in double (butterfly) and V.e as 16
//     key-strided partials + butterfly; the chunks combined in order by their weights
//     exp(m - max) in double: total = sum(sum * weight), output = sum fmaf(V.e, (float)(weight
//     / total), .);
//   * exp / erf: this file's own double routines (Cody-Waite + Taylor; two Chebyshev
//     interpolants), rounded to f32 once.
//
// The reference computes the same steps through ggml (src/mg/lm.h:152-259, src/nn.h:186-191,
// src/ac/transformer.h:28-38, src/mg/sampling.h:32-105).
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <stdexcept>
#include <type_traits>
#include <string>

#include "kernels.h"

namespace mgx {

// ------------------------------------------------------------------------------------
// scalar helpers
// ------------------------------------------------------------------------------------
__device__ __forceinline__ float h2f(uint16_t h) { return __half2float(__ushort_as_half(h)); }
__device__ __forceinline__ uint16_t f2h(float f) { return __half_as_ushort(__float2half_rn(f)); }

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

// erf: two Chebyshev interpolants in monomial form (erf_coeffs.py derives them from 40-digit
// values): |x| < 1: x * P(2x^2 - 1), P of degree 11; 1 <= |x| < 4: 1 - Q(|x| * 2/3 - 5/3), Q
// (erfc on [1, 4]) of degree 20; +-1 beyond. Absolute error below 1.5e-15 and 1.3e-12. The
// coefficients are compile-time constants: the unrolled Horner loops take them as immediates
// (an array in constant memory cost a cold scalar load in every GELU epilogue).
constexpr double ERF_P[12] = {
    0x1.ee51eb23cb7ebp-1, -0x1.1fd162921520ep-3, 0x1.454368017b319p-6,
    -0x1.2b902b7b26e28p-9, 0x1.c82aa24968f47p-13, -0x1.263991d3aca15p-16,
    0x1.4866394fa4c3ep-20, -0x1.429e4c163b13bp-24, 0x1.1ad503d95b599p-28,
    -0x1.c02cc0da54c52p-33, 0x1.4424c09b26e7bp-37, -0x1.2d4c29f5686cbp-42};
constexpr double ERF_Q[21] = {
    0x1.aab859b20b140p-12, -0x1.ac44a2cdb3c80p-9, 0x1.9180586b55ae8p-7,
    -0x1.cdb9fd59ee319p-6, 0x1.65964ef5668ffp-5, -0x1.7c8c5ebf7f0ccp-5,
    0x1.0521f53919ddep-5, -0x1.2faaceec90308p-7, -0x1.b5d2183e391e9p-8,
    0x1.3b371adacbf70p-7, -0x1.29d400459d61ep-8, -0x1.ca1cf08ac8d5dp-12,
    0x1.df3c4bd10ee4ep-10, -0x1.e7099cc2c7d56p-11, -0x1.d14ddd0a26b51p-15,
    0x1.3dc0c2909a110p-12, -0x1.e193532b72642p-14, -0x1.3af7b90db0f1ap-15,
    0x1.17a5709f8fe8ap-15, 0x1.048f70bb1e4f4p-20, -0x1.e180cb94805c1p-19};

__device__ __forceinline__ double derf(double x) {
    const double ax = __builtin_fabs(x);
    if (ax < 1.0) {
        const double t = __builtin_fma(2.0 * x, x, -1.0);
        double p = ERF_P[11];
#pragma unroll
        for (int n = 10; n >= 0; --n) p = __builtin_fma(p, t, ERF_P[n]);
        return x * p;
    }
    if (ax >= 4.0) return x > 0 ? 1.0 : -1.0;
    const double t = __builtin_fma(ax, 0x1.5555555555555p-1, -0x1.aaaaaaaaaaaabp+0);
    double p = ERF_Q[20];
#pragma unroll
    for (int n = 19; n >= 0; --n) p = __builtin_fma(p, t, ERF_Q[n]);
    const double r = 1.0 - p;
    return x > 0 ? r : -r;
}

// ggml_gelu_erf: 0.5*x*(1+erf(x/sqrt 2)) in f32 (lm.h:203). For |a| >= 4, 1 - |erf(a)| <
// 1.6e-8 is below half an ulp of 1.0f, so the f32 erf is exactly +-1 and derf is skipped.
__device__ __forceinline__ float gelu_erf(float x) {
    const float a = x * 0.70710678118654752440f;
    const float e = __builtin_fabsf(a) >= 4.0f ? (a > 0.0f ? 1.0f : -1.0f) : (float)derf((double)a);
    return 0.5f * x * (1.0f + e);
}

// Lane l gets v[l ^ OFF], every lane of the wave active: the xor exchange of __shfl_xor without
// its LDS crossbar round trip -- quad permutes for 1 and 2, two row shifts and a select for 4
// and 8, the gfx950 permlane swaps for 16 and 32 (swapping a register with itself leaves each
// lane's partner in one of the two results).
template <int OFF> __device__ __forceinline__ uint32_t xor_lane_u(uint32_t v) {
    const int lane = (int)(threadIdx.x & 63);
    if constexpr (OFF == 32) {
        auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        return lane < 32 ? r[1] : r[0];
    } else if constexpr (OFF == 16) {
        auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        return (lane & 16) ? r[0] : r[1];
    } else if constexpr (OFF == 1) {
        return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xf, 0xf, true);   // quad_perm [1,0,3,2]
    } else if constexpr (OFF == 2) {
        return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xf, 0xf, true);   // quad_perm [2,3,0,1]
    } else {
        static_assert(OFF == 4 || OFF == 8, "xor offsets 1 .. 32");
        const uint32_t up = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x100 + OFF, 0xf, 0xf, true);
        const uint32_t dn = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x110 + OFF, 0xf, 0xf, true);
        return (lane & OFF) ? dn : up;
    }
}
template <int OFF> __device__ __forceinline__ float xor_lane(float v) {
    return __uint_as_float(xor_lane_u<OFF>(__float_as_uint(v)));
}
template <int OFF> __device__ __forceinline__ int xor_lane(int v) { return (int)xor_lane_u<OFF>((uint32_t)v); }
template <int OFF> __device__ __forceinline__ double xor_lane(double v) {
    const uint64_t b = __double_as_longlong(v);
    const uint32_t lo = xor_lane_u<OFF>((uint32_t)b), hi = xor_lane_u<OFF>((uint32_t)(b >> 32));
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}
// v = op(v, v[l ^ off]) for off = OFF, OFF / 2, .., 1: the xor butterfly (each pair computes
// op on the same two operands, so for a commutative op every lane ends with the same value)
template <int OFF, typename T, typename Op> __device__ __forceinline__ T xor_reduce(T v, Op op) {
    v = op(v, xor_lane<OFF>(v));
    if constexpr (OFF > 1) return xor_reduce<OFF / 2>(v, op);
    else return v;
}
__device__ __forceinline__ float fmax_sel(float a, float b) { return a > b ? a : b; }
__device__ __forceinline__ float fmin_sel(float a, float b) { return a < b ? a : b; }

// Butterfly over the 64 lanes of a wave: lane l < off adds lane l+off, off = 32..1.
__device__ __forceinline__ float fold64(float v) {
    return xor_reduce<32>(v, [](float a, float b) { return a + b; });
}
__device__ __forceinline__ double fold64d(double v) {
    return xor_reduce<32>(v, [](double a, double b) { return a + b; });
}

// Q8_0 activation quantization of one element per lane; lanes 32k..32k+31 form one block.
// Writes q and (from the block's first lane) the fp16-rounded scale widened to f32.
__device__ __forceinline__ void quant_q8_lane(float v, int lane, int8_t* qdst, float* ddst) {
    const float amax = xor_reduce<16>(__builtin_fabsf(v), fmax_sel);
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    *qdst = (int8_t)__builtin_roundf(v * id);
    if ((lane & 31) == 0) *ddst = h2f(f2h(d));
}

// Byte offset of element i of column col in a block-major Q8 buffer of `stride` elements per
// column: columns go in groups of 16 (group col / 16 at stride * 16 bytes), and in a group block
// i / 32 holds 512 bytes in matrix-core operand order [g = (i % 32) / 8][col % 16][i % 8].
__device__ __forceinline__ size_t bm_off(int col, int i, int stride) {
    return (size_t)(col >> 4) * stride * 16 + (size_t)(i >> 5) * 512 + ((i >> 3) & 3) * 128 + (col & 15) * 8 + (i & 7);
}
// Index of the scale of element i's block: [group][block][col % 16].
__device__ __forceinline__ size_t bm_doff(int col, int i, int stride) {
    return (size_t)(col >> 4) * (stride / 32) * 16 + (size_t)(i >> 5) * 16 + (col & 15);
}

// The KV-cache column a QKV launch's column n appends to: its own column in the caller's
// numbering, or that modulo kv_cols when several columns share caches (a multi-position prefill).
__device__ __forceinline__ int kv_col(const GemvArgs& a, int n) {
    const int c = a.col0 + n;
    return a.kv_cols ? c % a.kv_cols : c;
}

// Writes element i (of a column) in the activation form the consumer's weights want.
__device__ __forceinline__ void put_act(const ActBuf& a, int col, int i, float v, int lane) {
    if (a.kind == ACT_Q8 && a.bm)
        quant_q8_lane(v, lane, a.q + bm_off(col, i, a.stride), a.d + bm_doff(col, i, a.stride));
    else if (a.kind == ACT_Q8) quant_q8_lane(v, lane, a.q + (size_t)col * a.stride + i, a.d + (size_t)col * (a.stride / 32) + i / 32);
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

// one block per (256 elements, request): request r's columns r*cols_per_req.. all get its sum
__global__ __launch_bounds__(256) void k_embed(EmbedArgs a) {
    const int i = blockIdx.x * 256 + threadIdx.x, r = blockIdx.y;
    if (i >= a.dim) return;
    const int p = a.pos[r];
    const float tab = a.table[(size_t)p * a.dim + i];
    const int32_t* ids = a.ids + (size_t)r * a.ids_req_stride;
    float e = 0.0f;
    for (int q = 0; q < a.n_q; ++q) {
        const int id = ids[(size_t)q * a.ids_stride + (p - a.ids_base)];
        const float v = mat_elem(a.emb[q], id, i);
        e = q == 0 ? v : e + v;
    }
    const float x = tab + e;
    for (int n = r * a.cols_per_req; n < (r + 1) * a.cols_per_req && n < a.ncol; ++n) a.x[(size_t)n * a.dim + i] = x;
}

__global__ __launch_bounds__(64) void k_advance(int* pos, int* live, const ReqParams* par, int n) {
    const int r = threadIdx.x;
    if (r >= n) return;
    if (!live) { pos[r] = pos[r] + 1; return; }
    if (!live[r]) return;
    const int np = pos[r] + 1;
    if (np + 1 >= par[r].steps) { live[r] = 0; pos[r] = 0; }
    else pos[r] = np;
}

__global__ __launch_bounds__(64) void k_slot_open(int* pos, int* live, ReqParams* par, int* nc, int r, ReqParams p,
                                                  int n_ctx) {
    if (threadIdx.x != 0) return;
    pos[r] = 0; live[r] = 1; par[r] = p; nc[r] = n_ctx;
}

__global__ __launch_bounds__(256) void k_add_bias(float* y, const float* b, int n, int ncol) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n * ncol) return;
    y[i] = y[i] + b[i % n];
}

// ------------------------------------------------------------------------------------
// GEMV: y[col][r] = W[r] . act[col] for up to 4 columns per launch.
//
// Layout: G lanes own a row (64/G rows per wave, WAVES waves per block); lane t of a row owns
// the row's partials p = t, t+G, ... and partial p accumulates units p, p+64, ... in order (a
// unit is a 32-element block for Q8_0 / Q4_0, 8 elements for F16 / F32), so the 64-partial
// butterfly's levels off >= G fold inside the lane and only off < G cross lanes.
//
// Issue order: the activation source (f32 columns, or the consumer-form activation), then
// every weight unit of the lane, then the residual -- vector-memory completions are counted
// in order, so the prologue only waits for its own loads. The prologue (LayerNorm /
// conversion / copy) builds the activation columns in LDS; the barriers wait for LDS only,
// so the dots start while later weight units are still arriving.
// ------------------------------------------------------------------------------------
constexpr int GEMV_KA = 4;   // 16-byte activation chunks per thread issued up front (PRO_ACT)

// lane l gets v[l + OFF] (OFF < 16: row-local DPP shift; 16 / 32: gfx950 permlane swaps);
// lanes whose source falls outside get garbage -- callers only use lanes that stay inside.
template <int OFF> __device__ __forceinline__ float take_up(float v) {
    if constexpr (OFF == 32) {
        auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        return __uint_as_float(r[1]);
    } else if constexpr (OFF == 16) {
        auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        return __uint_as_float(r[1]);
    } else {
        return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x100 + OFF, 0xf, 0xf, true));
    }
}
template <int OFF> __device__ __forceinline__ double take_up_d(double v) {
    const uint64_t b = __double_as_longlong(v);
    const float lo = take_up<OFF>(__uint_as_float((uint32_t)b));
    const float hi = take_up<OFF>(__uint_as_float((uint32_t)(b >> 32)));
    return __longlong_as_double((long long)(((uint64_t)__float_as_uint(hi) << 32) | __float_as_uint(lo)));
}
// lane l gets v[l - OFF] inside its 16-lane row
template <int OFF> __device__ __forceinline__ float take_dn(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x110 + OFF, 0xf, 0xf, true));
}
// Butterfly p[l] += p[l + off], off = G/2 .. 1: lane 0 of each G-lane group ends with the
// group's value (the butterfly's lane-0 result).
template <int G> __device__ __forceinline__ float fold_to0(float v) {
    if constexpr (G >= 64) v = v + take_up<32>(v);
    if constexpr (G >= 32) v = v + take_up<16>(v);
    if constexpr (G >= 16) v = v + take_up<8>(v);
    if constexpr (G >= 8) v = v + take_up<4>(v);
    if constexpr (G >= 4) v = v + take_up<2>(v);
    if constexpr (G >= 2) v = v + take_up<1>(v);
    return v;
}
// 64-lane double butterfly, result broadcast from lane 0
__device__ __forceinline__ double fold64d_b(double v) {
    v = v + take_up_d<32>(v);
    v = v + take_up_d<16>(v);
    v = v + take_up_d<8>(v);
    v = v + take_up_d<4>(v);
    v = v + take_up_d<2>(v);
    v = v + take_up_d<1>(v);
    const uint64_t b = __double_as_longlong(v);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)b), hi = __builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}
// max over each 8-lane group, to the group's first lane; then to all 8 lanes
__device__ __forceinline__ float grp8_max_to0(float v) {
    float o = take_up<1>(v); v = v > o ? v : o;
    o = take_up<2>(v); v = v > o ? v : o;
    o = take_up<4>(v); v = v > o ? v : o;
    return v;
}
__device__ __forceinline__ float grp8_bcast(float v, int lane) {
    float s = take_dn<1>(v); v = (lane & 1) ? s : v;
    s = take_dn<2>(v); v = (lane & 2) ? s : v;
    s = take_dn<4>(v); v = (lane & 4) ? s : v;
    return v;
}
// Loads of data read once per step and too large to stay cached (the K / V rows and the
// weights: GBs per step): non-temporal, so they do not evict what the step reads again
// (activations, positions, attention partials). Measured: c5 +7 %, c4 +3 % frames/s.
typedef float nt_f4 __attribute__((ext_vector_type(4)));
typedef int nt_i4 __attribute__((ext_vector_type(4)));
typedef unsigned nt_u2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ int4 ld_stream_i4(const void* p) {
    const nt_i4 v = __builtin_nontemporal_load((const nt_i4*)p);
    return make_int4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 ld_stream_u2(const void* p) {
    const nt_u2 v = __builtin_nontemporal_load((const nt_u2*)p);
    return make_uint2(v.x, v.y);
}
__device__ __forceinline__ float4 ld_stream(const float4* p) {
    const nt_f4 v = __builtin_nontemporal_load((const nt_f4*)p);
    return make_float4(v.x, v.y, v.z, v.w);
}

// Workgroup barrier for LDS traffic only: global loads in flight are not waited for.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Launch timing (profiled launches only): a launch's slot holds STAMP_SUB sub-slots of
// {earliest start, latest end} on the GPU's constant-rate wall clock. Block b publishes its end
// into sub-slot b mod STAMP_SUB once its waves are done, and the first STAMP_SUB blocks (the
// first dispatched, so the earliest start is among them) their start: at most a few atomics
// per address, so the stamps do not serialize behind each other (64 sub-slots with every block
// stamping added several us to a launch of 9000 blocks). The host takes the min / max over the
// sub-slots: the span a kernel tracer reports as the launch's duration.
__device__ __forceinline__ unsigned long long stamp_begin(const unsigned long long* p) {
    return p ? (unsigned long long)wall_clock64() : 0ull;
}
__device__ __forceinline__ unsigned stamp_block() {
    return blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
}
__device__ __forceinline__ unsigned long long* stamp_sub(unsigned long long* p) {
    return p + 2 * (stamp_block() % STAMP_SUB);
}
__device__ __forceinline__ void stamp_start(unsigned long long* p, unsigned long long t0) {
    if (stamp_block() < (unsigned)STAMP_SUB) atomicMin(stamp_sub(p), t0);
}
__device__ __forceinline__ void stamp_end(unsigned long long* p, unsigned long long t0) {
    if (!p) return;
    __syncthreads();
    if (threadIdx.x == 0) {
        stamp_start(p, t0);
        atomicMax(stamp_sub(p) + 1, (unsigned long long)wall_clock64());
    }
}

struct LdsAct {
    int8_t* q;     // Q8 [col][in]  (bm_col >= 0: global block-major of stride in, column bm_col)
    float* d;      // Q8 [col][in/32]
    uint16_t* h;   // F16 [col][in]
    float* f;      // F32 [col][in]
    int in;
    int bm_col;
};

template <int WT> struct WUnit;
// NT: the launch reads these weights once (it covers every column of the step): non-temporal.
// Launches in column pairs re-read them right after, from the caches.
template <> struct WUnit<T_Q8_0> {
    int4 a, b;
    uint16_t d;
    template <bool NT> __device__ __forceinline__ void load(const DevMat& m, int r, int u) {
        const int8_t* p = (const int8_t*)m.q + (size_t)r * m.in + u * 32;
        const uint16_t* pd = m.d + (size_t)r * (m.in / 32) + u;
        if constexpr (NT) { a = ld_stream_i4(p); b = ld_stream_i4(p + 16); d = __builtin_nontemporal_load(pd); }
        else { a = *(const int4*)p; b = *(const int4*)(p + 16); d = *pd; }
    }
};
template <> struct WUnit<T_Q4_0> {
    int4 a;
    uint16_t d;
    template <bool NT> __device__ __forceinline__ void load(const DevMat& m, int r, int u) {
        const uint8_t* p = (const uint8_t*)m.q + (size_t)r * (m.in / 2) + u * 16;
        const uint16_t* pd = m.d + (size_t)r * (m.in / 32) + u;
        if constexpr (NT) { a = ld_stream_i4(p); d = __builtin_nontemporal_load(pd); }
        else { a = *(const int4*)p; d = *pd; }
    }
};
template <> struct WUnit<T_F16> {
    int4 a;
    template <bool NT> __device__ __forceinline__ void load(const DevMat& m, int r, int u) {
        const uint16_t* p = (const uint16_t*)m.q + (size_t)r * m.in + u * 8;
        if constexpr (NT) a = ld_stream_i4(p);
        else a = *(const int4*)p;
    }
};
template <> struct WUnit<T_F32> {
    float4 a, b;
    template <bool NT> __device__ __forceinline__ void load(const DevMat& m, int r, int u) {
        const float* p = (const float*)m.q + (size_t)r * m.in + u * 8;
        a = *(const float4*)p; b = *(const float4*)(p + 4);
    }
};

// one unit of one activation column, read from LDS
template <int WT> struct ActUnit {
    int4 a, b;
    float d;
    __device__ __forceinline__ void load(const LdsAct& x, int n, int u) {
        const int8_t* xq = x.q + (size_t)n * x.in + u * 32;
        a = *(const int4*)xq; b = *(const int4*)(xq + 16);
        d = x.d[(size_t)n * (x.in / 32) + u];
    }
};
template <> struct ActUnit<T_F16> {
    int4 a;
    __device__ __forceinline__ void load(const LdsAct& x, int n, int u) { a = *(const int4*)(x.h + (size_t)n * x.in + u * 8); }
};
template <> struct ActUnit<T_F32> {
    float4 a, b;
    __device__ __forceinline__ void load(const LdsAct& x, int n, int u) {
        const float* xf = x.f + (size_t)n * x.in + u * 8;
        a = *(const float4*)xf; b = *(const float4*)(xf + 4);
    }
};

// Q8_0: exact integer block dot, term = (float)isum * (dw*dx).
__device__ __forceinline__ float dotr(const WUnit<T_Q8_0>& w, const ActUnit<T_Q8_0>& x, float p) {
    int s = __builtin_amdgcn_sdot4(w.a.x, x.a.x, 0, false);
    s = __builtin_amdgcn_sdot4(w.a.y, x.a.y, s, false);
    s = __builtin_amdgcn_sdot4(w.a.z, x.a.z, s, false);
    s = __builtin_amdgcn_sdot4(w.a.w, x.a.w, s, false);
    s = __builtin_amdgcn_sdot4(w.b.x, x.b.x, s, false);
    s = __builtin_amdgcn_sdot4(w.b.y, x.b.y, s, false);
    s = __builtin_amdgcn_sdot4(w.b.z, x.b.z, s, false);
    s = __builtin_amdgcn_sdot4(w.b.w, x.b.w, s, false);
    const float dd = h2f(w.d) * x.d;
    const float term = (float)s * dd;
    return p + term;
}
// Q4_0: sum((nib-8)*x) = sum(nib*x) - 8*sum(x), both exact integer dots.
__device__ __forceinline__ float dotr(const WUnit<T_Q4_0>& w, const ActUnit<T_Q4_0>& x, float p) {
    const uint32_t ws[4] = {(uint32_t)w.a.x, (uint32_t)w.a.y, (uint32_t)w.a.z, (uint32_t)w.a.w};
    const int xl[4] = {x.a.x, x.a.y, x.a.z, x.a.w}, xh[4] = {x.b.x, x.b.y, x.b.z, x.b.w};
    int s = 0, sx = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        s = __builtin_amdgcn_sdot4((int)(ws[k] & 0x0f0f0f0fu), xl[k], s, false);
        s = __builtin_amdgcn_sdot4((int)((ws[k] >> 4) & 0x0f0f0f0fu), xh[k], s, false);
        sx = __builtin_amdgcn_sdot4(0x01010101, xl[k], sx, false);
        sx = __builtin_amdgcn_sdot4(0x01010101, xh[k], sx, false);
    }
    const int isum = s - 8 * sx;
    const float dd = h2f(w.d) * x.d;
    const float term = (float)isum * dd;
    return p + term;
}
// F16 weights x fp16-rounded activations: products exact in f32, fmaf in element order.
__device__ __forceinline__ float dotr(const WUnit<T_F16>& w, const ActUnit<T_F16>& x, float p) {
    const uint32_t w32[4] = {(uint32_t)w.a.x, (uint32_t)w.a.y, (uint32_t)w.a.z, (uint32_t)w.a.w};
    const uint32_t x32[4] = {(uint32_t)x.a.x, (uint32_t)x.a.y, (uint32_t)x.a.z, (uint32_t)x.a.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        p = __builtin_fmaf(h2f((uint16_t)(w32[e] & 0xffffu)), h2f((uint16_t)(x32[e] & 0xffffu)), p);
        p = __builtin_fmaf(h2f((uint16_t)(w32[e] >> 16)), h2f((uint16_t)(x32[e] >> 16)), p);
    }
    return p;
}
__device__ __forceinline__ float dotr(const WUnit<T_F32>& w, const ActUnit<T_F32>& x, float p) {
    p = __builtin_fmaf(w.a.x, x.a.x, p); p = __builtin_fmaf(w.a.y, x.a.y, p);
    p = __builtin_fmaf(w.a.z, x.a.z, p); p = __builtin_fmaf(w.a.w, x.a.w, p);
    p = __builtin_fmaf(w.b.x, x.b.x, p); p = __builtin_fmaf(w.b.y, x.b.y, p);
    p = __builtin_fmaf(w.b.z, x.b.z, p); p = __builtin_fmaf(w.b.w, x.b.w, p);
    return p;
}

template <int WT>
__host__ __device__ constexpr int unit_elems() { return (WT == T_Q8_0 || WT == T_Q4_0) ? 32 : 8; }

__host__ __device__ inline size_t lds_act_bytes(int wt, int ncol, int in) {
    if (wt == T_Q8_0 || wt == T_Q4_0) return (size_t)ncol * in + (size_t)ncol * (in / 32) * 4;
    if (wt == T_F16) return (size_t)ncol * in * 2;
    return (size_t)ncol * in * 4;
}

// Sum of 256 per-thread partials red[0..255] in butterfly order (off 128 and 64 from LDS,
// 32..1 in-wave); every wave computes it and every lane gets it.
__device__ __forceinline__ double fold256(const double* red, int lane) {
    const double r = (red[lane] + red[lane + 128]) + (red[lane + 64] + red[lane + 192]);
    return fold64d_b(r);
}

// LayerNorm (transformer.h:28-38) or plain conversion of one f32 column into the activation
// form, in LDS, by a group of 256 threads (column n of the launch; each column has its own
// group). Thread i owns partial i: float4 groups i, i+256, ... of the column, summed in
// element order in double; the 256 partials are folded by the butterfly. Then (x - mean) *
// (1/sqrtf(var + eps)) * w + b per element, and quantization (each 32-element block is 8
// consecutive lanes). red: 512 doubles of LDS for this column.
template <int WT, int KG, bool LN>
__device__ __forceinline__ void prologue(const GemvArgs& a, const LdsAct& x, double* red, int n, int tid, int lane,
                                         const float4 (&xr)[KG], const float4 (&wr)[KG], const float4 (&br)[KG]) {
    const int in = a.w.in, nf = in / 4, nb = in / 32;
    float4 u[KG];
#pragma unroll
    for (int j = 0; j < KG; ++j) u[j] = tid + 256 * j < nf ? xr[j] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (LN) {
        double s = 0.0;
#pragma unroll
        for (int j = 0; j < KG; ++j) {
            s = s + (double)u[j].x; s = s + (double)u[j].y; s = s + (double)u[j].z; s = s + (double)u[j].w;
        }
        red[tid] = s;
        lds_barrier();
        const float mean = (float)(fold256(red, lane) / (double)in);
        double s2 = 0.0;
#pragma unroll
        for (int j = 0; j < KG; ++j) {
            float4 d = u[j];
            d.x = d.x - mean; d.y = d.y - mean; d.z = d.z - mean; d.w = d.w - mean;
            u[j] = d;
            if (tid + 256 * j < nf) {
                s2 = s2 + (double)(d.x * d.x); s2 = s2 + (double)(d.y * d.y);
                s2 = s2 + (double)(d.z * d.z); s2 = s2 + (double)(d.w * d.w);
            }
        }
        red[256 + tid] = s2;
        lds_barrier();
        const float var = (float)(fold256(red + 256, lane) / (double)in);
        const float scale = 1.0f / __builtin_sqrtf(var + a.eps);
#pragma unroll
        for (int j = 0; j < KG; ++j) {
            float4 t = u[j];
            t.x = t.x * scale; t.y = t.y * scale; t.z = t.z * scale; t.w = t.w * scale;
            t.x = t.x * wr[j].x; t.y = t.y * wr[j].y; t.z = t.z * wr[j].z; t.w = t.w * wr[j].w;
            t.x = t.x + br[j].x; t.y = t.y + br[j].y; t.z = t.z + br[j].z; t.w = t.w + br[j].w;
            u[j] = t;
        }
    }
#pragma unroll
    for (int j = 0; j < KG; ++j) {
        const int f = tid + 256 * j;
        const float4 t = u[j];
        if (WT == T_Q8_0 || WT == T_Q4_0) {
            float amax = __builtin_fabsf(t.x);
            amax = amax > __builtin_fabsf(t.y) ? amax : __builtin_fabsf(t.y);
            amax = amax > __builtin_fabsf(t.z) ? amax : __builtin_fabsf(t.z);
            amax = amax > __builtin_fabsf(t.w) ? amax : __builtin_fabsf(t.w);
            amax = grp8_bcast(grp8_max_to0(amax), lane);
            const float d = amax / 127.0f;
            const float id = d != 0.0f ? 1.0f / d : 0.0f;
            const uint32_t word = (uint32_t)(uint8_t)(int8_t)__builtin_roundf(t.x * id)
                                | (uint32_t)(uint8_t)(int8_t)__builtin_roundf(t.y * id) << 8
                                | (uint32_t)(uint8_t)(int8_t)__builtin_roundf(t.z * id) << 16
                                | (uint32_t)(uint8_t)(int8_t)__builtin_roundf(t.w * id) << 24;
            if (f < nf && x.bm_col >= 0) {
                *(uint32_t*)(x.q + bm_off(x.bm_col, 4 * f, in)) = word;
                if ((lane & 7) == 0) x.d[bm_doff(x.bm_col, 4 * f, in)] = h2f(f2h(d));
            } else if (f < nf) {
                *(uint32_t*)(x.q + (size_t)n * in + 4 * f) = word;
                if ((lane & 7) == 0) x.d[(size_t)n * nb + f / 8] = h2f(f2h(d));
            }
        } else if (WT == T_F16) {
            if (f < nf) {
                const uint32_t lo = (uint32_t)f2h(t.x) | (uint32_t)f2h(t.y) << 16;
                const uint32_t hi = (uint32_t)f2h(t.z) | (uint32_t)f2h(t.w) << 16;
                *(uint2*)(x.h + (size_t)n * in + 4 * f) = make_uint2(lo, hi);
            }
        } else if (f < nf) {
            *(float4*)(x.f + (size_t)n * in + 4 * f) = t;
        }
    }
}

// Adapter on one output (row, column) of a projection (lora.h:50-83): lo = B[row] . (Ax)[col]
// as f32 with rank k -> partial (k>>3) mod 64 (fmaf in order) folded by the 64-wide butterfly
// (partials >= 8 are zero: the first three levels add +0.0f), times s; v = base + lo; DoRA
// rows v *= m[row] / norm[row]; strength blend base + (v - base) * strength.
__device__ __forceinline__ float adapt_from(const GemvArgs& a, const float* bp, const float* xp, float m, float norm,
                                            float base) {
    float part[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) part[l] = 0.0f;
    for (int k = 0; k < a.ad_rank; ++k) part[k >> 3] = __builtin_fmaf(bp[k], xp[k], part[k >> 3]);
#pragma unroll
    for (int l = 0; l < 8; ++l) part[l] = part[l] + 0.0f;
#pragma unroll
    for (int off = 4; off >= 1; off >>= 1)
#pragma unroll
        for (int l = 0; l < off; ++l) part[l] = part[l] + part[l + off];
    const float lo = part[0] * a.ad_scale;
    float v = base + lo;
    if (a.ad_m) {
        v = v * (m / norm);
        if (a.ad_strength != 1.0f) v = base + (v - base) * a.ad_strength;
    }
    return v;
}
__device__ __forceinline__ float adapt(const GemvArgs& a, int row, int col, float base) {
    return adapt_from(a, a.ad_B + (size_t)row * a.ad_rank, a.ad_ax + (size_t)col * a.ad_rank,
                      a.ad_m ? a.ad_m[row] : 1.0f, a.ad_m ? a.ad_norm[row] : 1.0f, base);
}

// U > 0: every lane owns exactly U units (units == G * U). U == 0: any unit count, a runtime
// loop in passes of 8 units per lane (needs G == 8 so a pass covers each partial once).
template <int WT, int NC, int G, int U, int PRO, int EPI, int WAVES, bool NTW>
__device__ __forceinline__ void gemv_body(const GemvArgs& a) {
    constexpr int M = 64 / G, R = WAVES * M, NT = 64 * WAVES;
    constexpr int IN = U > 0 ? unit_elems<WT>() * G * U : 2048;   // prologue size bound
    constexpr int KG = (IN + 1023) / 1024;
    static_assert(PRO == PRO_ACT || WAVES == 4 * NC, "the prologue gives each column 256 threads (256 partials)");
    static_assert(U > 0 || G == 8, "the runtime unit loop folds 8 units per lane per pass");
    static_assert(EPI != EPI_GELU_ACT || R % 32 == 0, "GELU blocks quantize whole 32-row blocks");
    extern __shared__ __align__(16) uint8_t lds[];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int t = lane % G, rl = lane / G;
    const int in = a.w.in, out = a.w.out, nb = in / 32, ncol = a.ncol;
    const int row = blockIdx.x * R + wave * M + rl;
    const int row_ld = row < out ? row : out - 1;
    LdsAct x;
    x.in = in;
    x.bm_col = -1;
    x.q = (int8_t*)lds; x.d = (float*)(lds + (size_t)NC * in); x.h = (uint16_t*)lds; x.f = (float*)lds;
    float* tile = (float*)(lds + lds_act_bytes(WT, NC, in));
    double* red = (double*)(lds + lds_act_bytes(WT, NC, in) + (size_t)NC * R * 4);

    // 0. the qkv epilogue's cache row per column, read before everything else so its latency
    //    hides behind the weights instead of following the dots
    int qpos[NC];
    if constexpr (EPI == EPI_QKV) {
#pragma unroll
        for (int n = 0; n < NC; ++n) qpos[n] = a.pos[(a.col0 + (n < ncol ? n : ncol - 1)) >> a.cshift];
    }
    // 1. activation source (prologue: thread group pcol = tid / 256 builds column pcol)
    const int pcol = tid >> 8, ptid = tid & 255;
    float4 xr[PRO == PRO_ACT ? 1 : KG], wr[PRO == PRO_ACT ? 1 : KG], br[PRO == PRO_ACT ? 1 : KG];
    int4 ch[GEMV_KA];
    int nchunks = 0, cq = 0;
    if constexpr (PRO != PRO_ACT) {
        const int nf = in / 4;
        const float4* xs = (const float4*)(a.x + (size_t)(pcol < ncol ? pcol : ncol - 1) * a.x_stride);
#pragma unroll
        for (int j = 0; j < KG; ++j) {
            const int f = ptid + 256 * j < nf ? ptid + 256 * j : nf - 1;
            xr[j] = xs[f];
            if (PRO == PRO_LN) { wr[j] = ((const float4*)a.ln_w)[f]; br[j] = ((const float4*)a.ln_b)[f]; }
        }
    } else {
        // the source columns are contiguous: q [col][in] (or h / f), then Q8 scales [col][in/32]
        const size_t bq = (WT == T_Q8_0 || WT == T_Q4_0) ? (size_t)ncol * in
                        : (size_t)ncol * in * (WT == T_F16 ? 2 : 4);
        const size_t bd = (WT == T_Q8_0 || WT == T_Q4_0) ? (size_t)ncol * nb * 4 : 0;
        cq = (int)(bq / 16);
        nchunks = cq + (int)(bd / 16);
        const int4* sq = (const int4*)((WT == T_Q8_0 || WT == T_Q4_0) ? (const void*)a.src.q
                          : (WT == T_F16 ? (const void*)a.src.h : (const void*)a.src.f));
        const int4* sd = (const int4*)a.src.d;
#pragma unroll
        for (int k = 0; k < GEMV_KA; ++k) {
            int c = tid + NT * k;
            c = c < nchunks ? c : nchunks - 1;
            const int4* p = c < cq ? sq + c : sd + (c - cq);
            ch[k] = *p;
        }
    }
    if constexpr (PRO != PRO_ACT) {
        // every wave's column loads enter the memory pipeline before any wave's weight loads
        asm volatile("s_barrier" ::: "memory");
    }
    // 2. weights
    WUnit<WT> w[U > 0 ? U : 1];
    if constexpr (U > 0) {
#pragma unroll
        for (int i = 0; i < U; ++i) w[i].template load<NTW>(a.w, row_ld, t + G * i);
    }
    // 3. residual
    float yo[NC];
    if constexpr (EPI == EPI_RESID) {
#pragma unroll
        for (int n = 0; n < NC; ++n) yo[n] = a.y[(size_t)(n < ncol ? n : ncol - 1) * a.y_stride + row_ld];
    }
    if constexpr (PRO != PRO_ACT) __builtin_amdgcn_sched_barrier(0);
    // 4. activation -> LDS
    if constexpr (PRO != PRO_ACT) {
        prologue<WT, KG, PRO == PRO_LN>(a, x, red + pcol * 512, pcol, ptid, lane, xr, wr, br);
    } else {
        // a clamped index loaded the last chunk, so its store rewrites that chunk's own bytes
#pragma unroll
        for (int k = 0; k < GEMV_KA; ++k) {
            const int c = tid + NT * k;
            ((int4*)lds)[c < nchunks ? c : nchunks - 1] = ch[k];
        }
        const int4* sq = (const int4*)((WT == T_Q8_0 || WT == T_Q4_0) ? (const void*)a.src.q
                          : (WT == T_F16 ? (const void*)a.src.h : (const void*)a.src.f));
        for (int c = tid + NT * GEMV_KA; c < nchunks; c += NT)
            ((int4*)lds)[c] = c < cq ? sq[c] : ((const int4*)a.src.d)[c - cq];
    }
    lds_barrier();
    // 5. dots
    float acc[NC][M];
#pragma unroll
    for (int n = 0; n < NC; ++n)
#pragma unroll
        for (int m = 0; m < M; ++m) acc[n][m] = 0.0f;
    if constexpr (U > 0) {
#pragma unroll
        for (int i = 0; i < U; ++i) {
            ActUnit<WT> xa[NC];
#pragma unroll
            for (int n = 0; n < NC; ++n) xa[n].load(x, n, t + G * i);
#pragma unroll
            for (int n = 0; n < NC; ++n) acc[n][i % M] = dotr(w[i], xa[n], acc[n][i % M]);
        }
    } else {
        const int units = in / unit_elems<WT>();
        const int upl = t < units ? (units - t + G - 1) / G : 0;   // units t + G*i of this lane
        for (int i0 = 0; i0 < upl; i0 += M) {
            WUnit<WT> wp[M];
#pragma unroll
            for (int ii = 0; ii < M; ++ii) {
                const int i = i0 + ii < upl ? i0 + ii : upl - 1;
                wp[ii].template load<NTW>(a.w, row_ld, t + G * i);
            }
#pragma unroll
            for (int ii = 0; ii < M; ++ii) {
                if (i0 + ii >= upl) break;
                const int u = t + G * (i0 + ii);
#pragma unroll
                for (int n = 0; n < NC; ++n) {
                    ActUnit<WT> xa;
                    xa.load(x, n, u);
                    acc[n][ii] = dotr(wp[ii], xa, acc[n][ii]);
                }
            }
        }
    }
    float v[NC];
#pragma unroll
    for (int n = 0; n < NC; ++n) {
#pragma unroll
        for (int h = M / 2; h >= 1; h >>= 1)
#pragma unroll
            for (int m = 0; m < h; ++m) acc[n][m] = acc[n][m] + acc[n][m + h];
        v[n] = fold_to0<G>(acc[n][0]);
    }
    if (a.ad_ax && t == 0 && row < out) {
#pragma unroll
        for (int n = 0; n < NC; ++n)
            if (n < ncol) v[n] = adapt(a, row, n, v[n]);
    }
    // 6. epilogue: lane 0 of each row group holds every column's value
    if constexpr (EPI == EPI_GELU_ACT) {
        // the block's R rows -> LDS tile -> GELU (one value per lane, spread over the waves)
        // -> activation form, one 32-row block per wave pass
        const int rb = wave * M + rl;
        if (t == 0) {
#pragma unroll
            for (int n = 0; n < NC; ++n) tile[n * R + rb] = v[n];
        }
        lds_barrier();
        constexpr int STRIDE = NT / (NC * R) > 0 ? NT / (NC * R) : 1;
        for (int i = tid; i < NC * R * STRIDE; i += NT)
            if (i % STRIDE == 0) tile[i / STRIDE] = gelu_erf(tile[i / STRIDE]);
        lds_barrier();
        const ActBuf& d = a.dst;
        const int base = blockIdx.x * R;
        for (int pr = wave; pr < ncol * (R / 32); pr += WAVES) {
            const int n = pr / (R / 32), bk = pr % (R / 32);
            const float g = lane < 32 ? tile[n * R + bk * 32 + lane] : 0.0f;
            const int o = base + bk * 32 + lane;
            if (d.kind == ACT_Q8) {
                int8_t qv;
                float dv;
                quant_q8_lane(g, lane, &qv, &dv);
                if (lane < 32 && d.bm) {
                    d.q[bm_off(n, o, d.stride)] = qv;
                    if (lane == 0) d.d[bm_doff(n, o, d.stride)] = dv;
                } else if (lane < 32) {
                    d.q[(size_t)n * d.stride + o] = qv;
                    if (lane == 0) d.d[(size_t)n * (d.stride / 32) + o / 32] = dv;
                }
            } else if (lane < 32) {
                if (d.kind == ACT_F16) d.h[(size_t)n * d.stride + o] = f2h(g);
                else d.f[(size_t)n * d.stride + o] = g;
            }
            if (a.dst_f && lane < 32) a.dst_f[(size_t)n * d.stride + o] = g;
        }
        return;
    }
    if (row >= out || t != 0) return;
#pragma unroll
    for (int n = 0; n < NC; ++n) {
        if (n >= ncol) break;
        const float r = v[n];
        if (EPI == EPI_STORE) { if (!a.gate || a.gate[a.col0 + n]) a.y[(size_t)n * a.y_stride + row] = r; }
        else if (EPI == EPI_RESID) { if (!a.gate || a.gate[a.col0 + n]) a.y[(size_t)n * a.y_stride + row] = yo[n] + r; }
        else {
            const int sec = row / a.dim, wi = row - sec * a.dim, head = wi >> 6, dm = wi & 63;
            if (sec == 0) a.y[(size_t)n * a.dim + wi] = r;
            else (sec == 1 ? a.k : a.v)[(((size_t)kv_col(a, n) * a.heads + head) * a.cap + qpos[n]) * 64 + dm] = r;
        }
    }
}

// ------------------------------------------------------------------------------------
// decode self-attention over keys [0, pos] (nn.h:186-191, no mask for one query)
// ------------------------------------------------------------------------------------
// acc + e * v per component (fmaf) where `take`, else acc unchanged: the same values as a
// branch around the fmaf, without one (the caller's e read is unconditional and in bounds)
__device__ __forceinline__ float4 fmaf4_if(bool take, float e, const float4& v, const float4& acc) {
    const float4 t = make_float4(__builtin_fmaf(e, v.x, acc.x), __builtin_fmaf(e, v.y, acc.y),
                                 __builtin_fmaf(e, v.z, acc.z), __builtin_fmaf(e, v.w, acc.w));
    return take ? t : acc;
}

// Sum over the 16 lanes of a lane group of 16 values per lane, by recursive halving: after
// the four levels lane t holds the sum of value t. Each value's additions follow the
// butterfly p[l] + p[l+off], off = 8, 4, 2, 1 (the side that keeps a value adds its partner's).
__device__ __forceinline__ float halving16(float (&p)[16], int t) {
    float a[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const bool lo = (t & 8) == 0;
        const float recv = xor_lane<8>(lo ? p[i + 8] : p[i]);
        a[i] = (lo ? p[i] : p[i + 8]) + recv;
    }
    float b[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const bool lo = (t & 4) == 0;
        const float recv = xor_lane<4>(lo ? a[i + 4] : a[i]);
        b[i] = (lo ? a[i] : a[i + 4]) + recv;
    }
    float c[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const bool lo = (t & 2) == 0;
        const float recv = xor_lane<2>(lo ? b[i + 2] : b[i]);
        c[i] = (lo ? b[i] : b[i + 2]) + recv;
    }
    const bool lo = (t & 1) == 0;
    const float recv = xor_lane<1>(lo ? c[1] : c[0]);
    return (lo ? c[0] : c[1]) + recv;
}

// Sum over the 16 lanes of a lane group of 4 values per lane: levels 8 and 4 halve the values,
// 2 and 1 add in place. Lane t ends with value 2*((t>>3)&1) + ((t>>2)&1); each value's
// additions follow the butterfly p[l] + p[l+off], off = 8, 4, 2, 1.
__device__ __forceinline__ float halving4(const float (&p)[4], int t) {
    const bool lo8 = (t & 8) == 0;
    const float a0 = (lo8 ? p[0] : p[2]) + xor_lane<8>(lo8 ? p[2] : p[0]);
    const float a1 = (lo8 ? p[1] : p[3]) + xor_lane<8>(lo8 ? p[3] : p[1]);
    const bool lo4 = (t & 4) == 0;
    float b = (lo4 ? a0 : a1) + xor_lane<4>(lo4 ? a1 : a0);
    b = b + xor_lane<2>(b);
    return b + xor_lane<1>(b);
}

// The 16 key-strided partials of a chunk's V.e, lane l of a wave holding partials (l >> 4) + 4k
// for k = 0..3 (P[k]) and dimensions 4 (l & 15) .. + 3: the butterfly off 8 and 4 in registers,
// 2 and 1 across lanes 32 and 16 apart; lanes 0-15 end with the chunk's 64 outputs.
__device__ __forceinline__ float4 fold_partials16(const float4 (&P)[4]) {
    float4 a0 = make_float4(P[0].x + P[2].x, P[0].y + P[2].y, P[0].z + P[2].z, P[0].w + P[2].w);
    const float4 a1 = make_float4(P[1].x + P[3].x, P[1].y + P[3].y, P[1].z + P[3].z, P[1].w + P[3].w);
    a0 = make_float4(a0.x + a1.x, a0.y + a1.y, a0.z + a1.z, a0.w + a1.w);
    a0.x = a0.x + take_up<32>(a0.x); a0.y = a0.y + take_up<32>(a0.y);
    a0.z = a0.z + take_up<32>(a0.z); a0.w = a0.w + take_up<32>(a0.w);
    a0.x = a0.x + take_up<16>(a0.x); a0.y = a0.y + take_up<16>(a0.y);
    a0.z = a0.z + take_up<16>(a0.z); a0.w = a0.w + take_up<16>(a0.w);
    return a0;
}

// One 64-key chunk of one (head, column): 256 threads. Every load is issued up front (keys past
// the position re-read the last key: a cache hit, never a stale row): K as 16 lanes per key
// (four dims each), key 16*it + 4*wave + g for it = 0..3; V as 16 key-strided partials p =
// tid / 16 (keys p, p + 16, p + 32, p + 48) by 16 dimension quads. Scores: 16 four-dim fmaf
// partials folded by the butterfly, times the scale. The chunk's max m; e = expf(s - m) (0 past
// the position) in LDS; the chunk's sum of e in double by the 64-wide butterfly; o = sum e v as
// the 16 key-strided fmaf partials folded by the butterfly. Writes o [64], m and the sum; a
// chunk wholly past the column's position writes nothing (the combine reads only chunks that
// exist).
__global__ __launch_bounds__(256) void k_attn_chunk(AttnArgs a) {
    const unsigned long long t0 = stamp_begin(a.stamp);
    const int c = blockIdx.x, h = blockIdx.y, n = blockIdx.z, j0 = c * ATT_CHUNK;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, t = lane & 15;
    const size_t head = (size_t)n * a.heads + h;
    const size_t kvh = ((size_t)(a.kv_cols ? n % a.kv_cols : n) * a.heads + h) * a.cap * 64 + (size_t)j0 * 64;
    const float* K = a.k + kvh;
    const float* V = a.v + kvh;
    __shared__ float red_f[4];
    __shared__ float el[ATT_CHUNK];
    __shared__ float4 vred[16][16];
    // The chunk's 64 rows are loaded before the position is known (they lie inside the cache's
    // rows, which cover whole 256-key spans); rows past the position only ever enter masked
    // lanes, so their contents never reach a result.
    const float4 q = ((const float4*)(a.q + (size_t)n * a.dim + h * 64))[t];
    float4 kv[4];
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const float4* p = (const float4*)(K + (size_t)(it * 16 + wave * 4 + g) * 64) + t;
        kv[it] = ld_stream(p);
    }
    const int pv = tid >> 4, dq = tid & 15;
    float4 vv[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const float4* p = (const float4*)(V + (size_t)(pv + 16 * m) * 64) + dq;
        vv[m] = ld_stream(p);
    }
    const int u = a.pos[n >> a.cshift] + 1;
    if (j0 >= u) {
        if (a.stamp && threadIdx.x == 0) stamp_start(a.stamp, t0);
        return;
    }
    const int uc = u - j0 < ATT_CHUNK ? u - j0 : ATT_CHUNK;
    float pr[4];
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        float v = __builtin_fmaf(q.x, kv[it].x, 0.0f);
        v = __builtin_fmaf(q.y, kv[it].y, v);
        v = __builtin_fmaf(q.z, kv[it].z, v);
        pr[it] = __builtin_fmaf(q.w, kv[it].w, v);
    }
    // lanes t .. t ^ 3 hold key 16 * (2*((t>>3)&1) + ((t>>2)&1)) + 4 * wave + g
    const int jt = (2 * ((t >> 3) & 1) + ((t >> 2) & 1)) * 16 + wave * 4 + g;
    const float sc = halving4(pr, t) * a.scale;
    float mx = jt < uc ? sc : -__builtin_inff();
    mx = xor_reduce<32>(mx, fmax_sel);
    if (lane == 0) red_f[wave] = mx;
    lds_barrier();
    float m = red_f[0];
#pragma unroll
    for (int w = 1; w < 4; ++w) m = m > red_f[w] ? m : red_f[w];
    if ((t & 3) == 0) el[jt] = jt < uc ? dexpf(sc - m) : 0.0f;
    lds_barrier();
    // keys past the position keep the running value (a select: every e is in LDS, 0 past the
    // position, so no lane branches around its read)
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int mm = 0; mm < 4; ++mm) {
        const int j = pv + 16 * mm;
        acc = fmaf4_if(j < uc, el[j], vv[mm], acc);
    }
    vred[pv][dq] = acc;
    const double sum = wave == 0 ? fold64d_b((double)el[lane]) : 0.0;
    lds_barrier();
    if (wave == 0) {
        float4 P[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) P[k] = vred[g + 4 * k][t];
        const float4 o = fold_partials16(P);
        if (lane < 16) ((float4*)(a.opart + (head * a.max_chunks + c) * 64))[lane] = o;
        if (lane == 0) {
            a.cmax[head * a.max_chunks + c] = m;
            a.csum[head * a.max_chunks + c] = sum;
        }
    }
    if (a.stamp && threadIdx.x == 0) stamp_start(a.stamp, t0);
}

// Butterfly over 16 values in registers: v[i] += v[i + off], off = 8, 4, 2, 1 -- the tree that
// halving4 (the scores) and fold_partials16 (the V.e partials) apply across lanes.
__device__ __forceinline__ float tree16(float (&v)[16]) {
#pragma unroll
    for (int off = 8; off >= 1; off >>= 1)
#pragma unroll
        for (int i = 0; i < off; ++i) v[i] = v[i] + v[i + off];
    return v[0];
}

// Prefill attention, columns sharing caches (kv_cols > 0: a prefill group's positions, column n
// on cache n % kv_cols): one block of ATT_PF_WAVES waves per (64-key chunk, head, cache, group of
// ATT_PF_COLS query columns) stages the chunk's K and V in LDS once; wave w then serves, in pass
// p, query columns 2 (p WAVES + w) and the next of the group together (every K and V read feeds
// both; the q rows come by scalar loads). Each column's
// chunk result is the same arithmetic as k_attn_chunk's, term for term: lane j takes key j --
// the 16 four-dim fmaf partials of q.k in a register butterfly (halving4's tree), times the
// scale, the wave's max over the keys inside the column's position, e = expf(s - m), the double
// sum of e by the 64-wide butterfly with key j in lane j -- then lane d takes dimension d: the
// 16 key-strided partials (keys p, p + 16, p + 32, p + 48 by fmaf in order) in
// fold_partials16's tree. A chunk wholly past a column's position writes nothing for it.
__global__ __launch_bounds__(64 * ATT_PF_WAVES) void k_attn_prefill(AttnArgs a) {
    const unsigned long long t0 = stamp_begin(a.stamp);
    constexpr int KS = 68;   // padded K row: 8 lanes' float4 reads hit distinct banks
    constexpr int NT = 64 * ATT_PF_WAVES;
    __shared__ __align__(16) float Ks[ATT_CHUNK * KS];
    __shared__ __align__(16) float Vs[ATT_CHUNK * 64];
    __shared__ __align__(16) float es[ATT_PF_WAVES][2][64];
    // block L -> (item, query group): the groups of one item (chunk, head, cache) are blocks
    // L, L + 8, L + 16, .. -- one XCD (blocks go to the 8 XCDs in turn), dispatched together, so
    // the chunk comes from HBM once and from that XCD's L2 for the other groups
    const int groups = ((a.ncol + a.kv_cols - 1) / a.kv_cols + ATT_PF_COLS - 1) / ATT_PF_COLS, L = (int)blockIdx.x;
    const int item = (L / (8 * groups)) * 8 + (L & 7), grp = (L >> 3) % groups;
    const int nch = a.nch;
    if (item >= nch * a.heads * a.kv_cols) return;
    const int c = item % nch, h = (item / nch) % a.heads, kc = item / (nch * a.heads), j0 = c * ATT_CHUNK;
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int nq = (a.ncol - kc + a.kv_cols - 1) / a.kv_cols;   // columns kc, kc + kv_cols, ..
    const size_t kvh = ((size_t)kc * a.heads + h) * a.cap * 64 + (size_t)j0 * 64;
    // the chunk's rows lie inside the cache's whole 256-key spans; rows past a column's
    // position only ever enter masked lanes
    constexpr int PER = ATT_CHUNK * 16 / NT;
    float4 kr[PER], vr[PER];
#pragma unroll
    for (int m = 0; m < PER; ++m) {
        kr[m] = ((const float4*)(a.k + kvh))[tid + NT * m];
        vr[m] = ((const float4*)(a.v + kvh))[tid + NT * m];
    }
#pragma unroll
    for (int m = 0; m < PER; ++m) {
        const int f = tid + NT * m, row = f >> 4, c4 = f & 15;
        *(float4*)(Ks + row * KS + c4 * 4) = kr[m];
        *(float4*)(Vs + row * 64 + c4 * 4) = vr[m];
    }
    lds_barrier();
    // the columns' q rows are the same for every lane: scalar loads (read-only during the
    // kernel, hence the constant address space) into SGPRs, no LDS broadcast per use
    typedef const float __attribute__((address_space(4)))* qrow_t;
    for (int ps = 0; ps < ATT_PF_PASSES; ++ps) {
    // the pass's two columns (one past the group's end repeats the last and is not written)
    const int i0 = grp * ATT_PF_COLS + 2 * (ps * ATT_PF_WAVES + wave);
    if (i0 >= nq) break;
    const int na = kc + a.kv_cols * i0, nb = kc + a.kv_cols * (i0 + 1 < nq ? i0 + 1 : i0);
    const qrow_t qa_p = (qrow_t)(a.q + (size_t)na * a.dim + h * 64);
    const qrow_t qb_p = (qrow_t)(a.q + (size_t)nb * a.dim + h * 64);
    const int ua = a.pos[na >> a.cshift] + 1, ub = a.pos[nb >> a.cshift] + 1;
    const bool la = j0 < ua, lb = i0 + 1 < nq && j0 < ub;
    if (la || lb) {
        // keys inside each column's position (0: a column without this chunk)
        const int uca = la ? (ua - j0 < ATT_CHUNK ? ua - j0 : ATT_CHUNK) : 0;
        const int ucb = lb ? (ub - j0 < ATT_CHUNK ? ub - j0 : ATT_CHUNK) : 0;
        // the lane's key row in registers, then each column's 16 partials in turn
        float4 k4[16];
#pragma unroll
        for (int t = 0; t < 16; ++t) k4[t] = ((const float4*)(Ks + lane * KS))[t];
        float Pa[16], Pb[16];
        const auto qk = [&](qrow_t qp, float (&P)[16]) {
#pragma unroll
            for (int t = 0; t < 16; ++t) {
                float v = __builtin_fmaf(qp[4 * t], k4[t].x, 0.0f);
                v = __builtin_fmaf(qp[4 * t + 1], k4[t].y, v);
                v = __builtin_fmaf(qp[4 * t + 2], k4[t].z, v);
                P[t] = __builtin_fmaf(qp[4 * t + 3], k4[t].w, v);
            }
        };
        qk(qa_p, Pa);
        qk(qb_p, Pb);
        const float sa = tree16(Pa) * a.scale, sb = tree16(Pb) * a.scale;
        const float ma = xor_reduce<32>(lane < uca ? sa : -__builtin_inff(), fmax_sel);
        const float mb = xor_reduce<32>(lane < ucb ? sb : -__builtin_inff(), fmax_sel);
        const float ea = lane < uca ? dexpf(sa - ma) : 0.0f, eb = lane < ucb ? dexpf(sb - mb) : 0.0f;
        es[wave][0][lane] = ea;
        es[wave][1][lane] = eb;
        const double suma = fold64d_b((double)ea), sumb = fold64d_b((double)eb);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // the wave's e rows, before any lane reads them
        // keys past a position take no part: whole chunks run without a per-key test (a test
        // per key made each V read its own branch and LDS round trip); otherwise each column
        // keeps its running value by a select
        float Aa[16], Ab[16];
#pragma unroll
        for (int p = 0; p < 16; ++p) { Aa[p] = 0.0f; Ab[p] = 0.0f; }
        const auto pv = [&](auto whole) {
#pragma unroll
            for (int mm = 0; mm < 4; ++mm) {
#pragma unroll
                for (int p4 = 0; p4 < 4; ++p4) {
                    const float4 ea4 = ((const float4*)es[wave][0])[4 * mm + p4];   // keys 16 mm + 4 p4 .. + 3
                    const float4 eb4 = ((const float4*)es[wave][1])[4 * mm + p4];
                    const float eav[4] = {ea4.x, ea4.y, ea4.z, ea4.w}, ebv[4] = {eb4.x, eb4.y, eb4.z, eb4.w};
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const int p = 4 * p4 + k, j = 16 * mm + p;
                        const float v = Vs[j * 64 + lane];
                        const float ta = __builtin_fmaf(eav[k], v, Aa[p]), tb = __builtin_fmaf(ebv[k], v, Ab[p]);
                        Aa[p] = (decltype(whole)::value || j < uca) ? ta : Aa[p];
                        Ab[p] = (decltype(whole)::value || j < ucb) ? tb : Ab[p];
                    }
                }
            }
        };
        if (uca == ATT_CHUNK && ucb == ATT_CHUNK) pv(std::true_type{});
        else pv(std::false_type{});
        const float oa = tree16(Aa), ob = tree16(Ab);
        if (la) {
            const size_t hc = ((size_t)na * a.heads + h) * a.max_chunks + c;
            a.opart[hc * 64 + lane] = oa;
            if (lane == 0) { a.cmax[hc] = ma; a.csum[hc] = suma; }
        }
        if (lb) {
            const size_t hc = ((size_t)nb * a.heads + h) * a.max_chunks + c;
            a.opart[hc * 64 + lane] = ob;
            if (lane == 0) { a.cmax[hc] = mb; a.csum[hc] = sumb; }
        }
    }
    }
    if (a.stamp && threadIdx.x == 0) stamp_start(a.stamp, t0);
}

// The chunks of one (head, column) combined: lane c holds chunk c; M = max m_c, w_c =
// exp((double)m_c - M), total = the 64-wide butterfly of S_c * w_c (zeros past the column's
// chunks), f_c = (float)(w_c / total); lane d then sums fmaf(o_c[d], f_c, .) over the chunks in
// order. The head's 64 outputs go to the out-projection's activation.
// MC: the launch's chunk count (the 64-key chunks of its largest key count); chunks past the
// column's position take no part.
template <int MC>
__global__ __launch_bounds__(64) void k_attn_combine(AttnArgs a) {
    const int h = blockIdx.x, n = blockIdx.y, lane = threadIdx.x;
    const size_t head = (size_t)n * a.heads + h, hc = head * a.max_chunks;
    // every chunk slot of the launch is loaded before the position is known; slots past the
    // column's chunks are never used
    const int cl = lane < MC ? lane : MC - 1;
    const float mc0 = a.cmax[hc + cl];
    const double sc0 = a.csum[hc + cl];
    const float* op = a.opart + hc * 64 + lane;
    float o[MC];
#pragma unroll
    for (int k = 0; k < MC; ++k) o[k] = op[(size_t)k * 64];
    const int u = a.pos[n >> a.cshift] + 1, nch = (u + ATT_CHUNK - 1) / ATT_CHUNK;
    const bool live = lane < nch;
    const float mc = live ? mc0 : -__builtin_inff();
    float M = mc;
    M = xor_reduce<32>(M, fmax_sel);
    const double w = live ? dexp((double)mc - (double)M) : 0.0;
    const double total = fold64d_b(live ? sc0 * w : 0.0);
    const float f = live ? (float)(w / total) : 0.0f;
    float r = 0.0f;
#pragma unroll
    for (int k = 0; k < MC; ++k) {
        const float fk = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(f), k));
        r = k < nch ? __builtin_fmaf(o[k], fk, r) : r;
    }
    put_act(a.out, n, h * 64 + lane, r, lane);
    if (a.out_f) a.out_f[(size_t)n * a.dim + h * 64 + lane] = r;
    if (a.stamp && lane == 0) atomicMax(stamp_sub(a.stamp) + 1, (unsigned long long)wall_clock64());
}

// ------------------------------------------------------------------------------------
// cross-attention of the conditional stream over the projected memory (lm.h:181-199).
// The null stream's memory is zero, so its block output is exactly zero and is skipped.
// ------------------------------------------------------------------------------------
// One head's attention over nc <= 256 keys (the projected memory, or a T5 prompt) by 256
// threads: wave w takes the 64-key chunk w. Scores: 16 lanes per key (four dims each), key 64w +
// 4*it + g for it = 0..15, folded by the butterfly (after the halving reduce lane t holds it =
// t), times the scale, plus the bias row when given. Per chunk: its max m, e = expf(s - m), the
// sum of e in double by the 64-wide butterfly, V.e as 16 key-strided partials (lane l holds
// partials (l >> 4) + 4k, dims 4 (l & 15)..+3) folded by the butterfly. Wave 0 combines the
// chunks as the self-attention combine does. q: the head's 64 values. Output column r, elements
// h*64..h*64+63 of `out` (and of out_f when set); nc == 0 writes zeros.
__device__ __forceinline__ void xattn_head(const float* qh, const float* K, const float* V, int nc, float scale,
                                           const float* bias, const ActBuf& out, float* out_f, int dim, int h,
                                           int r) {
    __shared__ float cm[4];
    __shared__ double cs[4];
    __shared__ float4 co[4][16];
    __shared__ float el[256];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, t = lane & 15;
    const int j0 = wave * 64, uc = nc - j0 < 64 ? nc - j0 : 64;   // this wave's chunk holds uc keys
    const bool has = uc > 0;
    float4 kv[16], vv[16];
    const float4 q = ((const float4*)qh)[t];
#pragma unroll
    for (int it = 0; it < 16; ++it) {
        const int j = it * 4 + g, jl = j < uc ? j : uc - 1;
        kv[it] = has ? ((const float4*)(K + (size_t)(j0 + jl) * 64))[t] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int mm = 0; mm < 4; ++mm) {
            const int j = g + 4 * k + 16 * mm, jl = j < uc ? j : uc - 1;
            vv[4 * k + mm] = has ? ((const float4*)(V + (size_t)(j0 + jl) * 64))[t] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
    float p[16];
#pragma unroll
    for (int it = 0; it < 16; ++it) {
        float v = __builtin_fmaf(q.x, kv[it].x, 0.0f);
        v = __builtin_fmaf(q.y, kv[it].y, v);
        v = __builtin_fmaf(q.z, kv[it].z, v);
        p[it] = __builtin_fmaf(q.w, kv[it].w, v);
    }
    const int jt = 4 * t + g;   // this lane's key after the halving reduce
    float sc = halving16(p, t) * scale;
    if (bias && jt < uc) sc = sc + bias[j0 + jt];
    float m = jt < uc ? sc : -__builtin_inff();
    m = xor_reduce<32>(m, fmax_sel);
    el[j0 + jt] = jt < uc ? dexpf(sc - m) : 0.0f;
    lds_barrier();
    const double sum = fold64d_b((double)el[j0 + lane]);
    float4 P[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
        for (int mm = 0; mm < 4; ++mm) {
            const int j = g + 4 * k + 16 * mm;
            acc = fmaf4_if(j < uc, el[j0 + j], vv[4 * k + mm], acc);
        }
        P[k] = acc;
    }
    const float4 o = fold_partials16(P);
    if (lane < 16) co[wave][lane] = o;
    if (lane == 0) { cm[wave] = m; cs[wave] = sum; }
    lds_barrier();
    if (wave == 0) {
        const int nch = (nc + 63) / 64;
        const bool live = lane < nch;
        const float mcv = live ? cm[lane] : -__builtin_inff();
        float M = mcv;
        M = xor_reduce<32>(M, fmax_sel);
        const double w = live ? dexp((double)mcv - (double)M) : 0.0;
        const double total = fold64d_b(live ? cs[lane] * w : 0.0);
        const float f = live ? (float)(w / total) : 0.0f;
        const float* cof = (const float*)co;
        float res = 0.0f;
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) {
            if (cc >= nch) break;
            res = __builtin_fmaf(cof[cc * 64 + lane], __int_as_float(__builtin_amdgcn_readlane(__float_as_int(f), cc)), res);
        }
        const float v = nc > 0 ? res : 0.0f;
        put_act(out, r, h * 64 + lane, v, lane);
        if (out_f) out_f[(size_t)r * dim + h * 64 + lane] = v;
    }
}

// cross-attention of each request's conditional stream: one block per (head, request)
__global__ __launch_bounds__(256) void k_xattn(XAttnArgs a) {
    const unsigned long long t0 = stamp_begin(a.stamp);
    const int h = blockIdx.x, r = blockIdx.y, H = gridDim.x;
    const int nc = a.nc ? a.nc[r] : a.n_ctx;
    const size_t kr = a.shared_kv ? 0 : (size_t)r;
    const float* bias = a.bias ? a.bias + ((size_t)h * gridDim.y + r) * a.bias_stride : nullptr;
    xattn_head(a.q + (size_t)r * a.dim + h * 64, a.k + (kr * H + h) * a.n_ctx * 64,
                   a.v + (kr * H + h) * a.n_ctx * 64, nc, a.scale, bias, a.out, a.out_f, a.dim, h, r);
    stamp_end(a.stamp, t0);
}

// The hoisted cross K/V: projected [n_ctx][2*dim] -> K [H][rows][64], V [H][rows][64] (first n_ctx rows).
__global__ __launch_bounds__(256) void k_xkv_split(const float* kv, int n_ctx, int rows, int dim, float* k, float* v) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n_ctx * 2 * dim) return;
    const int t = i / (2 * dim), r = i - t * 2 * dim;
    const int sec = r / dim, w = r - sec * dim, head = w >> 6, d = w & 63;
    (sec == 0 ? k : v)[((size_t)head * rows + t) * 64 + d] = kv[i];
}

// ------------------------------------------------------------------------------------
// sampling: CFG mix + argmax / softmax, top-k, categorical (pipeline.cpp:264-294,
// sampling.h:32-105), one block per codebook
// ------------------------------------------------------------------------------------
constexpr int SMP_PER = MAX_CARD / 256;   // elements per thread

// Sequential double sum of n values held in LDS, in index order (one lane; loads batched
// ahead of the dependent adds).
__device__ __forceinline__ double seq_sum_d(const double* x, int n) {
    double t = 0.0;
    int i = 0;
    for (; i + 16 <= n; i += 16) {
        double b[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) b[k] = x[i + k];
#pragma unroll
        for (int k = 0; k < 16; ++k) t += b[k];
    }
    for (; i < n; ++i) t += x[i];
    return t;
}
__device__ __forceinline__ double seq_sum_f(const float* x, int n) {
    double t = 0.0;
    int i = 0;
    for (; i + 16 <= n; i += 16) {
        float b[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) b[k] = x[i + k];
#pragma unroll
        for (int k = 0; k < 16; ++k) t += (double)b[k];
    }
    for (; i < n; ++i) t += (double)x[i];
    return t;
}

// Double-double accumulation (h, l) += (b, bl): Knuth's two-sum of the high parts, the low
// parts added to its error, renormalized -- the sum stays within ~2^-100 of exact for the
// positive terms it is used on.
__device__ __forceinline__ void dd_add(double& h, double& l, double b, double bl) {
    const double s = h + b, bb = s - h;
    const double err = (h - (s - bb)) + (b - bb);
    const double t = err + (l + bl);
    h = s + t;
    l = t - (h - s);
}

// One xor level of the (largest value, lowest index) reduction, and of the double-double sum.
template <int OFF> __device__ __forceinline__ void argmax_level(float& best, int& bi) {
    const float ob = xor_lane<OFF>(best);
    const int oi = xor_lane<OFF>(bi);
    if (ob > best || (ob == best && oi < bi)) { best = ob; bi = oi; }
}
template <int OFF> __device__ __forceinline__ void dd_level(double& h, double& l) {
    const double oh = xor_lane<OFF>(h), ol = xor_lane<OFF>(l);
    dd_add(h, l, oh, ol);
}

// Block-wide inclusive scan of one int per thread (256 threads), through LDS.
__device__ __forceinline__ int block_scan_i(int v, int* tmp) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int o = __shfl_up(v, off, 64);
        if (lane >= off) v += o;
    }
    if (lane == 63) tmp[wave] = v;
    __syncthreads();
    int base = 0;
    for (int w = 0; w < wave; ++w) base += tmp[w];
    __syncthreads();
    return v + base;
}

__global__ __launch_bounds__(256) void k_sample(SampleArgs a) {
    const int q = blockIdx.x, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int C = a.card;
    __shared__ float lg[MAX_CARD];
    __shared__ double ex[MAX_CARD];
    __shared__ float pr[MAX_CARD];
    __shared__ int hist[256];
    __shared__ int itmp[8];
    __shared__ float red_f[4];
    __shared__ int red_i[4];
    __shared__ double red_d[4], dd_lo[4];
    __shared__ int tok_sh, pick_sh, exact_sh;
    __shared__ float inv_sh;
    __shared__ uint32_t prefix_sh;
    __shared__ int k_sh;
    const int r = blockIdx.y;
    const ReqParams par = a.par[r];
    const int offset = a.pos[r] + 1;
    // the whole block leaves together: a request that is idle or between its loop bounds
    if ((a.live && !a.live[r]) || offset < par.start || offset >= par.steps) return;
    const float cfg_coef = par.cfg_coef, temperature = par.temperature;
    const int use_sampling = par.use_sampling, top_k = par.top_k, guided = par.guided;
    const float* lr = a.logits + (size_t)r * a.cpr * a.n_q * C;
    const float* cond = lr + (size_t)q * C;
    const float* null_l = lr + (size_t)(a.n_q + q) * C;
    float* first = offset == par.start ? a.first_logits + (size_t)r * a.n_q * C : nullptr;
    float* stepl = a.step_logits ? a.step_logits + (((size_t)r * a.step_rows + (offset - par.start)) * a.n_q + q) * C : nullptr;
    const float* uniforms = a.uniforms + (size_t)r * a.seq_len * a.n_q;
    int32_t* seq = a.seq + (size_t)r * a.n_q * a.seq_len;
    const uint8_t* mask = a.mask + (size_t)r * a.mask_stride;
    // the step's mask byte, uniform and sequence slot, read up front (each used only after
    // several barriers; this block is the slot's only writer)
    const uint8_t mask_v = mask[(size_t)q * a.seq_len + offset];
    const float u_v = uniforms[(size_t)offset * a.n_q + q];
    const int32_t slot_v = seq[(size_t)q * a.seq_len + offset];
    for (int i = tid; i < C; i += 256) {
        float v = cond[i];
        if (guided) v = null_l[i] + (cond[i] - null_l[i]) * cfg_coef;
        lg[i] = v;
        if (first) first[(size_t)q * C + i] = v;
        if (stepl) stepl[i] = v;
    }
    __syncthreads();
    const bool timed = mask_v != 0;
    int token;
    if (!timed) token = a.special;
    else if (!use_sampling || !(temperature > 0.0f)) {
        // argmax, lowest index on ties
        float best = -__builtin_inff();
        int bi = 0x7fffffff;
        for (int i = tid; i < C; i += 256)
            if (lg[i] > best || (lg[i] == best && i < bi)) { best = lg[i]; bi = i; }
        argmax_level<32>(best, bi);
        argmax_level<16>(best, bi);
        argmax_level<8>(best, bi);
        argmax_level<4>(best, bi);
        argmax_level<2>(best, bi);
        argmax_level<1>(best, bi);
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
        // softmax_into: peak, double exps, total in index order, float scale
        float pk = -__builtin_inff();
        for (int i = tid; i < C; i += 256) pk = pk < lg[i] ? lg[i] : pk;
        pk = xor_reduce<32>(pk, [](float a, float b) { return a < b ? b : a; });
        if (lane == 0) red_f[wave] = pk;
        __syncthreads();
        pk = red_f[0];
        for (int w = 1; w < 4; ++w) pk = pk < red_f[w] ? red_f[w] : pk;
        // The reference's total is the sequential double sum of the e (sampling.h:47-51); only
        // (float)(1 / total) is used. The sum in double-double (error ~2^-100 relative) and the
        // sequential sum's error bound (n-1) u / (1 - (n-1) u) of it (all e >= 0) bracket the
        // sequential total; (float)(1.0 / t) is monotone in t, so when it is the same at both
        // ends of the bracket it is the reference's value. Otherwise (about 1e-5 of the rows)
        // one lane runs the sequential sum.
        double hs = 0.0, ls = 0.0;
        for (int i = tid; i < C; i += 256) {
            const double e = dexp(((double)lg[i] - (double)pk) / (double)temperature);
            ex[i] = e;
            pr[i] = (float)e;
            dd_add(hs, ls, e, 0.0);
        }
        dd_level<32>(hs, ls);
        dd_level<16>(hs, ls);
        dd_level<8>(hs, ls);
        dd_level<4>(hs, ls);
        dd_level<2>(hs, ls);
        dd_level<1>(hs, ls);
        if (lane == 0) { red_d[wave] = hs; dd_lo[wave] = ls; }
        __syncthreads();
        if (tid == 0) {
            double h = red_d[0], l = dd_lo[0];
            for (int w = 1; w < 4; ++w) dd_add(h, l, red_d[w], dd_lo[w]);
            const double sum = h + l, bound = (double)(C - 1) * 1.2e-16 * sum;
            const float a0 = (float)(1.0 / (sum + bound)), a1 = (float)(1.0 / (sum - bound));
            inv_sh = a0 == a1 ? a0 : (float)(1.0 / seq_sum_d(ex, C));
        }
        __syncthreads();
        for (int i = tid; i < C; i += 256) pr[i] = pr[i] * inv_sh;
        __syncthreads();
        const int k = top_k;
        if (k > 0 && k < C) {
            // top_k_filter: the k-th largest value counting repeats, by MSB-first radix select
            // over the bit patterns (non-negative floats order like their bits)
            if (tid == 0) { prefix_sh = 0; k_sh = k; }
            __syncthreads();
            for (int shift = 24; shift >= 0; shift -= 8) {
                // read before the barriers below; the one writer writes after them
                const uint32_t pre = prefix_sh;
                const int kk = k_sh;
                hist[tid] = 0;
                __syncthreads();
                const uint32_t hmask = shift == 24 ? 0u : (0xffffffffu << (shift + 8));
                for (int i = tid; i < C; i += 256) {
                    const uint32_t bits = __float_as_uint(pr[i]);
                    if ((bits & hmask) == (pre & hmask)) atomicAdd(&hist[(bits >> shift) & 255u], 1);
                }
                __syncthreads();
                // counts from the top bin down; the bin where the running count reaches k
                const int cnt = hist[255 - tid];
                const int incl = block_scan_i(cnt, itmp);
                if (incl >= kk && incl - cnt < kk) {
                    k_sh = kk - (incl - cnt);
                    prefix_sh = pre | ((uint32_t)(255 - tid) << shift);
                }
                __syncthreads();
            }
            const float cutoff = __uint_as_float(prefix_sh);
            float mn = __builtin_inff();
            for (int i = tid; i < C; i += 256) {
                if (pr[i] < cutoff) pr[i] = 0.0f;
                else if (pr[i] > 0.0f) mn = mn < pr[i] ? mn : pr[i];
            }
            // Every partial sum of these floats is exact in double when no survivor is below
            // 2^-29 (each is a multiple of 2^-52 and the sums stay below 2): any summation
            // order then gives the reference's sequential result.
            mn = xor_reduce<32>(mn, fmin_sel);
            if (lane == 0) red_f[wave] = mn;
            __syncthreads();
            if (tid == 0) {
                float m = red_f[0];
                for (int w = 1; w < 4; ++w) m = m < red_f[w] ? m : red_f[w];
                exact_sh = m >= 1.862645149230957e-09f;   // 2^-29
            }
            __syncthreads();
            double t = 0.0;
            if (exact_sh) {
                for (int i = tid; i < C; i += 256) t += (double)pr[i];
                t = xor_reduce<32>(t, [](double a, double b) { return a + b; });
                if (lane == 0) red_d[wave] = t;
                __syncthreads();
                if (tid == 0) inv_sh = (float)(1.0 / (red_d[0] + red_d[1] + red_d[2] + red_d[3]));
            } else if (tid == 0) {
                inv_sh = (float)(1.0 / seq_sum_f(pr, C));
            }
            __syncthreads();
            for (int i = tid; i < C; i += 256) pr[i] = pr[i] * inv_sh;
            __syncthreads();
        }
        // categorical(probs, 1.0): the first i whose running double sum exceeds u
        float mn = __builtin_inff();
        for (int i = tid; i < C; i += 256) if (pr[i] > 0.0f) mn = mn < pr[i] ? mn : pr[i];
        mn = xor_reduce<32>(mn, fmin_sel);
        if (lane == 0) red_f[wave] = mn;
        __syncthreads();
        if (tid == 0) {
            float m = red_f[0];
            for (int w = 1; w < 4; ++w) m = m < red_f[w] ? m : red_f[w];
            exact_sh = m >= 1.862645149230957e-09f;
            pick_sh = C - 1;
        }
        __syncthreads();
        const double target = (double)u_v * 1.0;
        if (exact_sh) {
            // thread t owns elements [SMP_PER*t, SMP_PER*t + SMP_PER); exact prefix sums
            double loc[SMP_PER];
            double s = 0.0;
#pragma unroll
            for (int e = 0; e < SMP_PER; ++e) {
                const int i = tid * SMP_PER + e;
                s += i < C ? (double)pr[i] : 0.0;
                loc[e] = s;
            }
            double incl = s;
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const double o = __shfl_up(incl, off, 64);
                if (lane >= off) incl += o;
            }
            if (lane == 63) red_d[wave] = incl;
            __syncthreads();
            double base = incl - s;
            for (int w = 0; w < wave; ++w) base += red_d[w];
            int found = 0x7fffffff;
#pragma unroll
            for (int e = SMP_PER - 1; e >= 0; --e) {
                const int i = tid * SMP_PER + e;
                if (i < C && base + loc[e] > target) found = i;
            }
            if (found != 0x7fffffff) atomicMin(&pick_sh, found);
        } else if (tid == 0) {
            double acc = 0.0;
            int pick = C - 1;
            for (int i = 0; i < C; ++i) {
                acc += (double)pr[i];
                if (acc > target) { pick = i; break; }
            }
            pick_sh = pick;
        }
        __syncthreads();
        token = pick_sh;
    }
    if (tid == 0 && slot_v == -1) seq[(size_t)q * a.seq_len + offset] = token;
}

// ------------------------------------------------------------------------------------
// repack: ggml blocks -> device layout. Q8_0 {d, q[32]} rows split into q[out][in] +
// d[out][in/32]; Q4_0 {d, qs[16]} into qs[out][in/2] + d. One thread per block.
// ------------------------------------------------------------------------------------
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

// ------------------------------------------------------------------------------------
// launchers
// ------------------------------------------------------------------------------------
void launch_embed(const EmbedArgs& a, hipStream_t s) {
    const int nreq = (a.ncol + a.cols_per_req - 1) / a.cols_per_req;
    hipLaunchKernelGGL(k_embed, dim3((a.dim + 255) / 256, nreq), dim3(256), 0, s, a);
}
void launch_advance(int* pos, int* live, const ReqParams* par, int n_req, hipStream_t s) {
    hipLaunchKernelGGL(k_advance, dim3(1), dim3(64), 0, s, pos, live, par, n_req);
}
__global__ __launch_bounds__(64) void k_set_positions(int* pos, int n, int p0) {
    for (int r = threadIdx.x; r < n; r += 64) pos[r] = p0 + r;
}
void launch_set_positions(int* pos, int n, int p0, hipStream_t s) {
    hipLaunchKernelGGL(k_set_positions, dim3(1), dim3(64), 0, s, pos, n, p0);
}
__global__ __launch_bounds__(64) void k_fill_i32(int* p, int n, int v) {
    for (int r = threadIdx.x; r < n; r += 64) p[r] = v;
}
void launch_fill_i32(int* p, int n, int v, hipStream_t s) {
    hipLaunchKernelGGL(k_fill_i32, dim3(1), dim3(64), 0, s, p, n, v);
}
void launch_slot_open(int* pos, int* live, ReqParams* par, int* nc, int r, const ReqParams& p, int n_ctx,
                      hipStream_t s) {
    hipLaunchKernelGGL(k_slot_open, dim3(1), dim3(64), 0, s, pos, live, par, nc, r, p, n_ctx);
}
void launch_add_bias(float* y, const float* b, int n, int ncol, hipStream_t s) {
    hipLaunchKernelGGL(k_add_bias, dim3((n * ncol + 255) / 256), dim3(256), 0, s, y, b, n, ncol);
}

// The arguments of the column group starting at column c0 of a0's columns: every per-column
// pointer advanced, the caller's numbering (col0) moved along; the QKV epilogue's caches stay
// (it maps col0 + n to its cache row).
__host__ __device__ __forceinline__ void gemv_advance(GemvArgs& a, const GemvArgs& a0, int c0) {
    a.x = a0.x ? a0.x + (size_t)c0 * a0.x_stride : nullptr;
    const auto adv = [c0](ActBuf& b, const ActBuf& b0) {
        if (b0.q) b.q = b0.q + (size_t)c0 * b0.stride;
        if (b0.d) b.d = b0.d + (size_t)c0 * (b0.stride / 32);
        if (b0.h) b.h = b0.h + (size_t)c0 * b0.stride;
        if (b0.f) b.f = b0.f + (size_t)c0 * b0.stride;
    };
    adv(a.src, a0.src);
    adv(a.dst, a0.dst);
    if (a0.dst_f) a.dst_f = a0.dst_f + (size_t)c0 * a0.dst.stride;
    if (a0.ad_ax) a.ad_ax = a0.ad_ax + (size_t)c0 * a0.ad_rank;
    a.col0 = a0.col0 + c0;
    if (a0.epi == EPI_QKV) a.y = a0.y + (size_t)c0 * a0.dim;
    else if (a0.y) a.y = a0.y + (size_t)c0 * a0.y_stride;
}

// blockIdx.y > 0 (F16 / F32 weights: a launch over several whole groups of NC columns): the
// group's arguments. Quantized weights launch column groups one by one (their multi-column
// steps go to the matrix cores), so their instances stay free of the per-group arithmetic.
template <int WT, int NC, int G, int U, int PRO, int EPI, int WAVES, bool NTW>
__global__ __launch_bounds__(64 * WAVES) void k_gemv(GemvArgs a0) {
    const unsigned long long t0 = stamp_begin(a0.stamp);
    // group 0 reads the kernel arguments in place; a later group's copy lives in private memory
    if constexpr (WT == T_F16 || WT == T_F32) {
        if (blockIdx.y) {
            GemvArgs a = a0;
            gemv_advance(a, a0, (int)blockIdx.y * NC);
            gemv_body<WT, NC, G, U, PRO, EPI, WAVES, NTW>(a);
        } else {
            gemv_body<WT, NC, G, U, PRO, EPI, WAVES, NTW>(a0);
        }
    } else {
        gemv_body<WT, NC, G, U, PRO, EPI, WAVES, NTW>(a0);
    }
    stamp_end(a0.stamp, t0);
}

// ------------------------------------------------------------------------------------
// multi-column Q8_0 GEMV on the matrix cores (3 to 16 activation columns)
// ------------------------------------------------------------------------------------
// The integer dot product of each 32-element block, for 16 rows x 16 columns, is one
// v_mfma_i32_16x16x32_i8 (exact: integer sums). The float terms (float)isum * (dw * dx) are
// then summed as every GEMV sums them: partial b mod 64 in increasing b, the 64 partials
// folded by the butterfly (offsets 32..1). Wave w of KW owns the partials p = w (mod KW), whose
// butterfly is a subtree of the full one: it visits them in the subtree's in-order (bit-
// reversed) order and merges finished subtrees as a binary counter does, which performs the
// same additions on the same operands; the KW subtree sums meet in LDS for the top levels.
// Lane (g, c) = (lane / 16, lane % 16) feeds row c / column c, bytes 8g..8g+7 of each block,
// and receives rows 4g..4g+3 of column c. Activations come in Q8 form from global memory;
// weight scales from the tile-transposed copy dt.
typedef int mf_v4i __attribute__((ext_vector_type(4)));

template <int BITS>
__host__ __device__ constexpr int bitrev(int j) {
    int r = 0;
    for (int k = 0; k < BITS; ++k) r |= ((j >> k) & 1) << (BITS - 1 - k);
    return r;
}
template <int N>
__host__ __device__ constexpr int ilog2() { return N <= 1 ? 0 : 1 + ilog2<N / 2>(); }

// One lane's A operand (16 rows x 32 of a block: row lane % 16, elements 8 (lane / 16) .. + 7).
// Q8_0: the 8 quants. Q4_0: one word whose byte m holds element m (low nibble) and element m + 4
// (high nibble), unpacked to int8 nib - 8 per byte ((x + 0x78) ^ 0x80 never carries out of a byte).
template <int WT> struct MfW;
template <> struct MfW<T_Q8_0> {
    using T = uint2;
    static __device__ __forceinline__ T load(const int8_t* qm, size_t i) { return ld_stream_u2((const uint2*)qm + i); }
    static __device__ __forceinline__ long op(T w) { return (long)(((unsigned long long)w.y << 32) | w.x); }
};
template <> struct MfW<T_Q4_0> {
    using T = uint32_t;
    static __device__ __forceinline__ T load(const int8_t* qm, size_t i) { return __builtin_nontemporal_load((const uint32_t*)qm + i); }
    static __device__ __forceinline__ long op(T w) {
        const uint32_t lo = ((w & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u;
        const uint32_t hi = (((w >> 4) & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u;
        return (long)(((unsigned long long)hi << 32) | lo);
    }
};

__device__ __forceinline__ void mf_opaque(uint2& v) { asm volatile("" : "+v"(v.x), "+v"(v.y)); }
__device__ __forceinline__ void mf_opaque(uint32_t& v) { asm volatile("" : "+v"(v)); }

template <int WT, int NB, int KW, int TILES, int EPI, bool WIDE>
__global__ __launch_bounds__(64 * KW) void k_gemv_mf(GemvArgs a) {
    constexpr int M = 64 / KW;                        // leaves (partials) per wave
    constexpr int LB = ilog2<M>();
    constexpr int S = NB >= 64 ? NB / 64 : 1;         // blocks per partial
    constexpr int NVL = NB >= 64 ? M : NB / KW;       // leaves with blocks: i < NVL
    constexpr int ROWS = 16 * TILES, NT = 64 * KW;
    static_assert(NB % KW == 0 && (NB < 64 || NB % 64 == 0), "unsupported width");
    static_assert(EPI != EPI_GELU_ACT || ROWS == 32, "GELU blocks quantize whole 32-row blocks");
    __shared__ float yg[WIDE ? MF_WIDE_GROUPS : 1][ROWS][17];   // WIDE: the block's column groups' sums
    // adapter operands: the tile's B rows, one column group's A x (rank <= 64), DoRA m and norm
    constexpr int AD_MAX = (ROWS + 16) * 64 + 2 * ROWS, AD_PER = (AD_MAX + 64 * KW - 1) / (64 * KW);
    __shared__ float adsh[AD_MAX];
    // the waves' subtree sums; WIDE launches alternate two buffers where LDS allows, so a group's
    // writes need no barrier behind the previous group's reads (the barrier after each group's
    // writes orders the reads of the buffer two groups back)
    constexpr int RED_FLOATS = KW * ROWS * 17;
    constexpr int NRED = WIDE && (2 * RED_FLOATS + MF_WIDE_GROUPS * ROWS * 17 + AD_MAX) * 4 <= 56 * 1024 ? 2 : 1;
    __shared__ float red[NRED][KW][ROWS][17];
    const unsigned long long t0 = stamp_begin(a.stamp);
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, g = lane >> 4, c16 = lane & 15;
    // WIDE (17 to MF_MAX_COLS columns): the block's column groups (blockIdx.y's share of the launch's)
    // one after another against one load of the weights, every group's epilogue after the last
    // (an adapter's operands staged group by group); else one group, epilogue in place
    const int row0 = blockIdx.x * ROWS, ncol = a.ncol;
    const int gpb = WIDE ? (((ncol + 15) >> 4) + gridDim.y - 1) / gridDim.y : 1;
    const int cg0 = WIDE ? blockIdx.y * gpb : 0;
    const int cg1 = WIDE ? (cg0 + gpb < ((ncol + 15) >> 4) ? cg0 + gpb : ((ncol + 15) >> 4)) : 1;
    if (cg0 >= cg1) return;   // (the launcher gives every block a group)
    const ActBuf& x = a.src;
    const int8_t* Wm = a.w.qm;
    // one 16-column group of the block-major source: stride * 16 quant bytes, stride / 2 scales
    const size_t gq = (size_t)x.stride * 16, gd = (size_t)(x.stride / 32) * 16;
    // widths up to 2048 prefetch the next group's activations during a group's reduction; wider
    // rows hold too many weight registers for that and load them at the group's start
    constexpr bool PREFETCH = NB < 192;
    // 1. every load of the wave, in visiting order (a leaf's weights, activations and scales
    //    together, so its products can start while later leaves are still loading)
    typename MfW<WT>::T wa[TILES][M][S];
    uint2 xb[M][S], dw[TILES][M][S];
    float xd[M][S];
    const auto load_x = [&](int grp) {
#pragma unroll
        for (int j = 0; j < M; ++j) {
            const int i = bitrev<LB>(j);
            if (i >= NVL) continue;
#pragma unroll
            for (int s = 0; s < S; ++s) {
                const int b = w + KW * i + 64 * s;
                xb[j][s] = *(const uint2*)(x.q + grp * gq + ((size_t)b * 64 + lane) * 8);
                xd[j][s] = x.d[grp * gd + (size_t)b * 16 + c16];
            }
        }
    };
#pragma unroll
    for (int j = 0; j < M; ++j) {
        const int i = bitrev<LB>(j);
        if (i >= NVL) continue;
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const int b = w + KW * i + 64 * s;
#pragma unroll
            for (int t = 0; t < TILES; ++t)
                wa[t][j][s] = MfW<WT>::load(Wm, ((size_t)(row0 / 16 + t) * NB + b) * 64 + lane);
            xb[j][s] = *(const uint2*)(x.q + cg0 * gq + ((size_t)b * 64 + lane) * 8);
            xd[j][s] = x.d[cg0 * gd + (size_t)b * 16 + c16];
#pragma unroll
            for (int t = 0; t < TILES; ++t)
                dw[t][j][s] = ld_stream_u2(a.w.dt + ((size_t)(row0 / 16 + t) * NB + b) * 16 + 4 * g);
        }
    }
    // adapter operands behind the weights (used only in the epilogue)
    const int ad_nb = a.ad_ax ? ROWS * a.ad_rank : 0, ad_nx = a.ad_ax ? ad_nb + (WIDE ? 16 : ncol) * a.ad_rank : 0;
    const int ad_n = ad_nx + (a.ad_ax && a.ad_m ? 2 * ROWS : 0);
    float adr[WIDE ? 1 : AD_PER];
    if (!WIDE && a.ad_ax) {
        // one unconditional load per slot: the address is selected, slots past the end re-read B[0]
#pragma unroll
        for (int k = 0; k < AD_PER; ++k) {
            const int e = tid + 64 * KW * k;
            const float* src = e < ad_nb ? a.ad_B + (size_t)row0 * a.ad_rank + e
                             : e < ad_nx ? a.ad_ax + (e - ad_nb)
                             : e >= ad_n ? a.ad_B
                             : e < ad_nx + ROWS ? a.ad_m + row0 + (e - ad_nx)
                             : a.ad_norm + row0 + (e - ad_nx - ROWS);
            adr[k] = *src;
        }
    }
    // the qkv epilogue's cache row of column tid (decode groups: staged in LDS with the adapter
    // operands; prefill groups read theirs in the epilogue)
    __shared__ int posl[16];
    int posr = 0;
    if (EPI == EPI_QKV && !WIDE) posr = a.pos[(a.col0 + (tid < ncol ? (tid & 15) : ncol - 1)) >> a.cshift];
    // the residual epilogue's x values of the outputs this thread finishes (decode groups)
    constexpr int RES_PER = (ROWS * 16 + NT - 1) / NT;
    float yres[RES_PER];
    if constexpr (EPI == EPI_RESID && !WIDE) {
#pragma unroll
        for (int k = 0; k < RES_PER; ++k) {
            const int idx = tid + NT * k, n = idx / ROWS, r = idx % ROWS;
            const int nc = idx < ROWS * 16 && n < ncol ? n : ncol - 1, row = row0 + r < a.w.out ? row0 + r : a.w.out - 1;
            yres[k] = a.y[(size_t)nc * a.y_stride + row];
        }
    }
    // keep every load above in flight together: the scheduler would otherwise sink each next
    // to its first use and pay the memory latency once per leaf
    __builtin_amdgcn_sched_barrier(0);
    // one output (row row0 + r, column n): the adapter, then the epilogue. (The caches' bases
    // are read once here: a per-lane choice between two argument fields would otherwise become
    // a per-lane load of the chosen field.)
    float* const kcache = a.k;
    float* const vcache = a.v;
    const auto finish = [&](int n, int r, float y, float yr) {
        const int row = row0 + r;
        const bool live = n < ncol;
        if (a.ad_ax && live)    // the staged A x holds column n's group (n < 16 when not WIDE)
            y = adapt_from(a, adsh + r * a.ad_rank, adsh + ad_nb + (n & 15) * a.ad_rank, a.ad_m ? adsh[ad_nx + r] : 1.0f,
                           a.ad_m ? adsh[ad_nx + ROWS + r] : 1.0f, y);
        if constexpr (EPI == EPI_GELU_ACT) {
            const float ge = gelu_erf(y);
            const ActBuf& d = a.dst;
            if (d.kind == ACT_Q8) {
                int8_t qv;
                float dv;
                quant_q8_lane(ge, lane, &qv, &dv);    // lanes 32k..32k+31: one column's 32 rows
                if (live && d.bm) {
                    d.q[bm_off(n, row, d.stride)] = qv;
                    if ((lane & 31) == 0) d.d[bm_doff(n, row, d.stride)] = dv;
                } else if (live) {
                    d.q[(size_t)n * d.stride + row] = qv;
                    if ((lane & 31) == 0) d.d[(size_t)n * (d.stride / 32) + row / 32] = dv;
                }
            } else if (live) {
                if (d.kind == ACT_F16) d.h[(size_t)n * d.stride + row] = f2h(ge);
                else d.f[(size_t)n * d.stride + row] = ge;
            }
            if (live && a.dst_f) a.dst_f[(size_t)n * d.stride + row] = ge;
        } else if (live && (EPI == EPI_QKV || !a.gate || a.gate[a.col0 + n])) {
            if (EPI == EPI_STORE) a.y[(size_t)n * a.y_stride + row] = y;
            else if (EPI == EPI_RESID) a.y[(size_t)n * a.y_stride + row] = (WIDE ? a.y[(size_t)n * a.y_stride + row] : yr) + y;
            else {
                const int sec = row / a.dim, wi = row - sec * a.dim, head = wi >> 6, dm = wi & 63;
                if (sec == 0) a.y[(size_t)n * a.dim + wi] = y;
                else (sec == 1 ? kcache : vcache)[(((size_t)kv_col(a, n) * a.heads + head) * a.cap +
                                                   (WIDE ? a.pos[(a.col0 + n) >> a.cshift] : posl[n])) * 64 + dm] = y;
            }
        }
    };
    // column groups one after another against the same weights (in registers)
    for (int cg = cg0;;) {
    if (WIDE && !PREFETCH && cg > cg0) {
        load_x(cg);
        __builtin_amdgcn_sched_barrier(0);
    }
    // 2. leaves in order, merged as a binary counter
    float4 lev[TILES][LB + 1];
#pragma unroll
    for (int j = 0; j < M; ++j) {
        const int i = bitrev<LB>(j);
        float4 leaf[TILES];
#pragma unroll
        for (int t = 0; t < TILES; ++t) leaf[t] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (i < NVL) {
#pragma unroll
            for (int s = 0; s < S; ++s) {
#pragma unroll
                for (int t = 0; t < TILES; ++t) {
                    const mf_v4i z = {0, 0, 0, 0};
                    const mf_v4i r = __builtin_amdgcn_mfma_i32_16x16x32_i8(
                        MfW<WT>::op(wa[t][j][s]),
                        (long)(((unsigned long long)xb[j][s].y << 32) | xb[j][s].x), z, 0, 0, 0);
                    const float dx = xd[j][s];
                    const float d0 = h2f((uint16_t)(dw[t][j][s].x & 0xffffu)) * dx;
                    const float d1 = h2f((uint16_t)(dw[t][j][s].x >> 16)) * dx;
                    const float d2 = h2f((uint16_t)(dw[t][j][s].y & 0xffffu)) * dx;
                    const float d3 = h2f((uint16_t)(dw[t][j][s].y >> 16)) * dx;
                    leaf[t].x = leaf[t].x + (float)r[0] * d0;
                    leaf[t].y = leaf[t].y + (float)r[1] * d1;
                    leaf[t].z = leaf[t].z + (float)r[2] * d2;
                    leaf[t].w = leaf[t].w + (float)r[3] * d3;
                }
            }
        }
#pragma unroll
        for (int t = 0; t < TILES; ++t) {
            float4 carry = leaf[t];
            int k = 0;
#pragma unroll
            for (; k < LB && ((j >> k) & 1); ++k) {
                carry.x = lev[t][k].x + carry.x; carry.y = lev[t][k].y + carry.y;
                carry.z = lev[t][k].z + carry.z; carry.w = lev[t][k].w + carry.w;
            }
            lev[t][k] = carry;
        }
    }
    // the next group's activations, behind this group's reduction (when the registers allow)
    if (WIDE && PREFETCH && cg + 1 < cg1) load_x(cg + 1);
    __builtin_amdgcn_sched_barrier(0);
    // 3. the KW subtree sums -> the top of the tree, one (row, column) per thread
#pragma unroll
    for (int t = 0; t < TILES; ++t) {
        red[cg & (NRED - 1)][w][16 * t + 4 * g + 0][c16] = lev[t][LB].x;
        red[cg & (NRED - 1)][w][16 * t + 4 * g + 1][c16] = lev[t][LB].y;
        red[cg & (NRED - 1)][w][16 * t + 4 * g + 2][c16] = lev[t][LB].z;
        red[cg & (NRED - 1)][w][16 * t + 4 * g + 3][c16] = lev[t][LB].w;
    }
    if constexpr (!WIDE) {
#pragma unroll
        for (int k = 0; k < AD_PER; ++k)
            if (tid + 64 * KW * k < ad_n) adsh[tid + 64 * KW * k] = adr[k];
        if (EPI == EPI_QKV && tid < 16) posl[tid] = posr;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < RES_PER; ++k) {
        const int idx0 = NT * k, idx = idx0 + tid;
        if (idx0 + (tid & ~63) >= ROWS * 16) break;    // whole waves past the tile
        const int n = idx / ROWS, r = idx % ROWS;
        float v[KW];
#pragma unroll
        for (int q = 0; q < KW; ++q) v[q] = red[cg & (NRED - 1)][q][r][n];
#pragma unroll
        for (int off = KW / 2; off >= 1; off >>= 1)
#pragma unroll
            for (int q = 0; q < off; ++q) v[q] = v[q] + v[q + off];
        if constexpr (WIDE) yg[cg - cg0][r][n] = v[0];
        else finish(n, r, v[0], (EPI == EPI_RESID) ? yres[k] : 0.0f);
    }
    if constexpr (!WIDE) break;
    if (++cg >= cg1) break;
    if constexpr (NRED == 1) __syncthreads();   // the next group rewrites red
    // the empty asm makes the weights look new to the next group, so their conversions (fp16
    // scales, Q4_0 nibbles) are not hoisted out of the loop into twice the registers; at the
    // loop's end, so the first group's products still start while its later loads are in flight
#pragma unroll
    for (int j = 0; j < M; ++j) {
        if (bitrev<LB>(j) >= NVL) continue;
#pragma unroll
        for (int s = 0; s < S; ++s)
#pragma unroll
            for (int t = 0; t < TILES; ++t) {
                mf_opaque(wa[t][j][s]);
                mf_opaque(dw[t][j][s]);
            }
    }
    }
    // 4. WIDE: every group's epilogues, once the weights' registers are free
    if constexpr (WIDE) {
        __syncthreads();
        if (!a.ad_ax) {
            for (int idx0 = 0; idx0 < (cg1 - cg0) * ROWS * 16; idx0 += NT) {
                const int idx = idx0 + tid;
                if (idx0 + (tid & ~63) >= (cg1 - cg0) * ROWS * 16) break;    // whole waves past the last group
                const int n = cg0 * 16 + idx / ROWS, r = idx % ROWS;
                finish(n, r, yg[(n >> 4) - cg0][r][n & 15], 0.0f);
            }
        } else {
            for (int g2 = cg0; g2 < cg1; ++g2) {
                // the group's adapter operands: the tile's B rows, its 16 columns' A x (0 past the
                // launch's columns), DoRA m and norm -- the layout the non-WIDE staging builds
                const int ax0 = g2 * 16 * a.ad_rank, axn = ncol * a.ad_rank;
                for (int e = tid; e < ad_n; e += NT)
                    adsh[e] = e < ad_nb ? a.ad_B[(size_t)row0 * a.ad_rank + e]
                            : e < ad_nx ? (ax0 + e - ad_nb < axn ? a.ad_ax[ax0 + e - ad_nb] : 0.0f)
                            : e < ad_nx + ROWS ? a.ad_m[row0 + (e - ad_nx)]
                            : a.ad_norm[row0 + (e - ad_nx - ROWS)];
                __syncthreads();
                for (int idx0 = 0; idx0 < ROWS * 16; idx0 += NT) {
                    const int idx = idx0 + tid;
                    if (idx0 + (tid & ~63) >= ROWS * 16) break;    // whole waves past the group
                    const int nl = idx / ROWS, r = idx % ROWS;
                    finish(g2 * 16 + nl, r, yg[g2 - cg0][r][nl], 0.0f);
                }
                __syncthreads();   // the next group rewrites the staged operands
            }
        }
    }
    stamp_end(a.stamp, t0);
}


// ---- GEMV launch: kernel choice by weight type, prologue / epilogue kind and unit count
template <int WT, int NC, int G, int U, int PRO, int EPI, int W, bool NTW>
static void gemv_go(const GemvArgs& a, hipStream_t s) {
    constexpr int R = W * (64 / G);
    const size_t lds = lds_act_bytes(WT, NC, a.w.in) + (size_t)NC * R * 4 + (PRO == PRO_ACT ? 0 : (size_t)NC * 512 * 8);
    hipLaunchKernelGGL((k_gemv<WT, NC, G, U, PRO, EPI, W, NTW>), dim3((a.w.out + R - 1) / R, a.ygroups > 1 ? a.ygroups : 1),
                       dim3(64 * W), lds, s, a);
}

// Tries (G, U, W) = the listed shapes whose G * U matches the row's unit count; else the
// runtime-loop kernel.
#define GEMV_TRY(G_, U_, W_) if (units == (G_) * (U_)) return gemv_go<WT, NC, G_, U_, PRO, EPI, W_, NTW>(a, s)


template <int WT, int NC, int PRO, int EPI, bool NTW> static void gemv_pick(const GemvArgs& a, hipStream_t s) {
    const int units = a.w.in / unit_elems<WT>();
    if constexpr (PRO == PRO_ACT) {
        if constexpr (WT == T_Q8_0 || WT == T_Q4_0) {
            // in = dim 1024 / 1536 / 2048: one wave of 4 rows a block (4x the blocks of 16-row
            // ones: 0.1-0.2 us faster at dim 1536); in = ff: 8 rows a block
            GEMV_TRY(16, 2, 1); GEMV_TRY(16, 3, 1); GEMV_TRY(16, 4, 1);
            GEMV_TRY(32, 4, 4); GEMV_TRY(32, 6, 4); GEMV_TRY(32, 8, 4);      // in = ff 4096 / 6144 / 8192
            GEMV_TRY(8, 2, 2);                                               // in = 512
        } else if constexpr (EPI == EPI_GELU_ACT) {
            // (F16 / F32 LayerNorm projections over prepared columns) the GELU epilogue takes
            // whole 32-row blocks: 8 lanes a row, 4 waves
            GEMV_TRY(8, 16, 4); GEMV_TRY(8, 8, 4); GEMV_TRY(8, 2, 4);
        } else if constexpr (WT == T_F16) {
            GEMV_TRY(8, 16, 2); GEMV_TRY(64, 8, 4); GEMV_TRY(8, 2, 2); GEMV_TRY(8, 8, 2);
        } else {
            GEMV_TRY(8, 2, 2); GEMV_TRY(8, 8, 2);
        }
    } else if constexpr (PRO == PRO_LN) {
        // 256 threads per column: 4 waves at one column, 8 at two; the GELU epilogue needs
        // 32-row blocks, so a one-column GELU launch takes 8 lanes a row
        constexpr int GL = (EPI == EPI_GELU_ACT && NC == 1) ? 8 : 16;
        if constexpr (WT == T_Q8_0 || WT == T_Q4_0) {
            GEMV_TRY(GL, 32 / GL, 4 * NC); GEMV_TRY(GL, 48 / GL, 4 * NC); GEMV_TRY(GL, 64 / GL, 4 * NC);
        } else if constexpr (WT == T_F16) {
            GEMV_TRY(GL, 128 / GL, 4 * NC); GEMV_TRY(8, 2, 4 * NC);
        } else {
            GEMV_TRY(8, 2, 4 * NC);
        }
    }
    if constexpr (PRO == PRO_ACT) gemv_go<WT, NC, 8, 0, PRO, EPI, 4, NTW>(a, s);
    else gemv_go<WT, NC, 8, 0, PRO, EPI, 4 * NC, NTW>(a, s);
}
#undef GEMV_TRY

template <int WT, int NC, bool NTW> static void gemv_nc(const GemvArgs& a, hipStream_t s) {
    if (a.pro == PRO_ACT) {
        // F16 / F32 LayerNorm projections over many columns take their columns prepared once
        // (k_prep) instead of per row block; every other activation-source site adds the residual
        if constexpr (WT == T_F16 || WT == T_F32) {
            if (a.epi == EPI_QKV) return gemv_pick<WT, NC, PRO_ACT, EPI_QKV, NTW>(a, s);
            if (a.epi == EPI_GELU_ACT) return gemv_pick<WT, NC, PRO_ACT, EPI_GELU_ACT, NTW>(a, s);
            if (a.epi == EPI_STORE) return gemv_pick<WT, NC, PRO_ACT, EPI_STORE, NTW>(a, s);
        }
        gemv_pick<WT, NC, PRO_ACT, EPI_RESID, NTW>(a, s);
    }
    else if (a.pro == PRO_F32) gemv_pick<WT, NC, PRO_F32, EPI_STORE, NTW>(a, s);
    else if (a.epi == EPI_QKV) gemv_pick<WT, NC, PRO_LN, EPI_QKV, NTW>(a, s);
    else if (a.epi == EPI_GELU_ACT) gemv_pick<WT, NC, PRO_LN, EPI_GELU_ACT, NTW>(a, s);
    else gemv_pick<WT, NC, PRO_LN, EPI_STORE, NTW>(a, s);
}
template <int WT, bool NTW> static void gemv_ncol(const GemvArgs& a, hipStream_t s) {
    if (a.ncol == 1) gemv_nc<WT, 1, NTW>(a, s);
    else if (a.ncol == 2) gemv_nc<WT, 2, NTW>(a, s);
    else if constexpr (WT == T_F16 || WT == T_F32) gemv_nc<WT, 4, NTW>(a, s);
    else throw std::logic_error("internal: a quantized vector GEMV of more than 2 columns");
}
// stream_w: the launch covers every column of the step, so its weights are read once and
// bypass the caches; launches over column groups of a wider step read them again right after.
template <int WT> static void gemv_wt(const GemvArgs& a, hipStream_t s) {
    if (a.stream_w) gemv_ncol<WT, true>(a, s);
    else gemv_ncol<WT, false>(a, s);
}
// Columns per vector-GEMV launch: 4 for F16 / F32 weights over more than 2 columns when the
// columns fit the block's LDS (those wide steps -- prompt groups, T5's tokens -- have no
// matrix-core path; each lane's weights then serve 4 columns, summed per column in the same
// order), else 2. A prologue launch gives each column 4 waves, so 4 columns halve its row
// blocks: it takes 4 only over 2048 rows and up, and the f32-source prologue never. Measured:
// activation-source launches T5 242 -> 283 encodes/s, small F16 prefill 254 -> 226 ms; the
// LayerNorm launches of 2048+ rows too 226 -> 204 ms; every prologue launch, T5 176.
static int gemv_step(const GemvArgs& a) {
    if (a.ncol <= 2 || (a.w.type != T_F16 && a.w.type != T_F32)) return 2;
    if (a.pro == PRO_F32 || (a.pro == PRO_LN && a.w.out < 2048)) return 2;
    // the columns, the epilogue tile (at most 128 rows a block) and the LayerNorm partials
    const size_t lds = lds_act_bytes(a.w.type, 4, a.w.in) + 4 * 128 * 4 + (a.pro == PRO_ACT ? 0 : 4 * 512 * 8);
    return lds <= 65536 ? 4 : 2;
}

// ---- matrix-core GEMV: (blocks per row, waves per 16-row tile) choices
static int mf_kw(int nb, int tiles_out, bool wide, bool gelu) {
    if (nb >= 256) return 8;   // 8192-wide rows: 16 waves would need more than 128 registers
    if (nb % 16) return 4;     // 128-wide rows (small test models)
    // decode batches (3-16 columns): 16 waves whatever the row count (c5's qkv: 6.8 -> 6.1 us,
    // 4 waves at 288 row tiles before); the wide GELU launch too (c4 ff.0: 19.2 -> 13.0 us,
    // 8 waves 14.8 at 64 columns; with 512-column groups 8 waves cost c4's prefill 2 ms more);
    // other wide launches 8 (c4 qkv 17.0 -> 11.0 us, c3 qkv 9.45 -> 8.7; 16 there: 11.8 at c3,
    // c5's prefill 694 -> 726 ms; at 512 columns 8 waves also beat 16 for fewer row tiles) but
    // the 6144-wide rows, whose 8-wave form needs 205 registers (c3 ff.2 58.2 us against 50.9;
    // prefill c3 29.3 -> 28.6 ms, c5 324.7 -> 319.1 with 16)
    if (!wide || gelu || nb == 192) return 16;
    return 8;
}
// widths 128 .. 6144 (8192 would need more than the 128 registers of a 1024-thread block)
static bool mf_width(int nb) {
    return nb == 4 || nb == 16 || nb == 32 || nb == 48 || nb == 64 || nb == 128 || nb == 192;
}
bool gemv_mf_ok(const GemvArgs& a) {
    const int rows = a.epi == EPI_GELU_ACT ? 32 : 16;
    return (a.w.type == T_Q8_0 || a.w.type == T_Q4_0) && a.w.dt && a.w.qm && a.pro == PRO_ACT && a.src.kind == ACT_Q8 &&
           a.src.bm &&
           a.src.stride == a.w.in &&
           a.ncol >= 3 && a.ncol <= MF_MAX_COLS && a.w.in % 32 == 0 &&
           (mf_width(a.w.in / 32) || (a.w.type == T_Q4_0 && a.w.in / 32 == 256)) && a.w.out % rows == 0 &&
           (a.epi != EPI_GELU_ACT || a.w.in <= 2048);
}
template <int WT, int NB, int KW, int TILES, int EPI> static void mf_go(const GemvArgs& a, hipStream_t s) {
    if (a.ncol > 16) {
        // the column groups over blockIdx.y, several per block (each block loads its tile's
        // weights once for its groups): up to MF_WIDE_GROUPS from 128 row tiles up, 4 below,
        // 2 up to 64 columns (a short prompt's group or an unguided view's tail). Measured
        // prefill at 64-column groups: 2 per block against 4 c3 76.6 -> 70.1 ms, c4 319 -> 288 ms
        // (1 per block 76.3, 327 ms), the GELU launch (32-row tiles) better at 4 (10.6 against
        // 12.9 ms at c3); at 128- and 256-column groups 4 per block beat 2 (c4 189.5 -> 186.6,
        // 165.1 -> 156.1 ms); at 512-column groups 8 beat 4 where the row tiles are 128 or more
        // (c4 138.7 -> 132.7 ms, c3 29.9 -> 29.2, c5 328.7 -> 324.4) and lost below that (8 for
        // every launch: c3 30.0 -> 30.4, c5 328.9 -> 337.4 -- their 96-tile launches then have
        // 384 blocks)
        const int groups = (a.ncol + 15) / 16, tiles = a.w.out / (16 * TILES);
        const int per = (EPI == EPI_GELU_ACT || groups > 4) ? (tiles >= 128 ? MF_WIDE_GROUPS : 4) : 2;
        const int split = (groups + per - 1) / per;
        hipLaunchKernelGGL((k_gemv_mf<WT, NB, KW, TILES, EPI, true>), dim3(tiles, split), dim3(64 * KW), 0, s, a);
    }
    else
        hipLaunchKernelGGL((k_gemv_mf<WT, NB, KW, TILES, EPI, false>), dim3(a.w.out / (16 * TILES)), dim3(64 * KW), 0, s, a);
}
template <int WT, int NB, int KW> static void mf_epi(const GemvArgs& a, hipStream_t s) {
    switch (a.epi) {
    case EPI_STORE: mf_go<WT, NB, KW, 1, EPI_STORE>(a, s); break;
    case EPI_RESID: mf_go<WT, NB, KW, 1, EPI_RESID>(a, s); break;
    case EPI_QKV: mf_go<WT, NB, KW, 1, EPI_QKV>(a, s); break;
    default: if constexpr (NB <= 64) mf_go<WT, NB, KW, 2, EPI_GELU_ACT>(a, s); break;
    }
}
template <int WT, int NB> static void mf_nb(const GemvArgs& a, hipStream_t s) {
    // mf_kw gives 4 only for NB not a multiple of 16, 16 only when it divides NB and NB < 256
    switch (mf_kw(NB, a.w.out / (a.epi == EPI_GELU_ACT ? 32 : 16), a.ncol > 16, a.epi == EPI_GELU_ACT)) {
    case 4: if constexpr (NB % 16 != 0) mf_epi<WT, NB, 4>(a, s); break;
    case 8: if constexpr (NB % 16 == 0) mf_epi<WT, NB, 8>(a, s); break;
    default: if constexpr (NB % 16 == 0 && NB < 256) mf_epi<WT, NB, 16>(a, s); break;
    }
}
template <int WT> static void mf_wt(const GemvArgs& a, hipStream_t s) {
    switch (a.w.in / 32) {
    case 4: mf_nb<WT, 4>(a, s); break;
    case 16: mf_nb<WT, 16>(a, s); break;
    case 32: mf_nb<WT, 32>(a, s); break;
    case 48: mf_nb<WT, 48>(a, s); break;
    case 64: mf_nb<WT, 64>(a, s); break;
    case 128: mf_nb<WT, 128>(a, s); break;
    case 192: mf_nb<WT, 192>(a, s); break;
    default: if constexpr (WT == T_Q4_0) mf_nb<WT, 256>(a, s); break;   // 4-bit weights: half the registers
    }
}
static void launch_gemv_mf(const GemvArgs& a, hipStream_t s) {
    if (a.w.type == T_Q4_0) mf_wt<T_Q4_0>(a, s);
    else mf_wt<T_Q8_0>(a, s);
}

// Vector GEMVs go in groups of gemv_step columns (every per-column pointer advanced by the
// group's offset).
void launch_gemv(const GemvArgs& a0, hipStream_t s) {
    if (gemv_mf_ok(a0)) {
        launch_gemv_mf(a0, s);
        return;
    }
    if (a0.pro == PRO_ACT && a0.src.bm) return;   // the caller checks gemv_mf_ok before making one
    const int step = gemv_step(a0), whole = a0.ncol / step;
    const bool grid_y = a0.w.type == T_F16 || a0.w.type == T_F32;
    // F16 / F32 weights: whole groups of `step` columns in one launch (blockIdx.y = the group:
    // one boundary for a prompt group's hundreds of columns), then a ragged tail in its own;
    // quantized weights one launch per group
    for (int c0 = 0; c0 < a0.ncol;) {
        GemvArgs a = a0;
        a.ygroups = grid_y && c0 == 0 && whole > 1 ? whole : 1;
        a.ncol = a0.ncol - c0 < step ? a0.ncol - c0 : step;
        a.stream_w = a0.ncol <= step ? 1 : 0;
        if (c0) gemv_advance(a, a0, c0);
        c0 += a.ncol * a.ygroups;
        switch (a.w.type) {
        case T_Q8_0: gemv_wt<T_Q8_0>(a, s); break;
        case T_Q4_0: gemv_wt<T_Q4_0>(a, s); break;
        case T_F16: gemv_wt<T_F16>(a, s); break;
        default: gemv_wt<T_F32>(a, s); break;
        }
    }
}
template <int MC>
static void launch_combine(const AttnArgs& a, int nch, hipStream_t s) {
    if constexpr (MC <= ATT_MAX_CHUNKS) {
        if (nch == MC) hipLaunchKernelGGL(k_attn_combine<MC>, dim3(a.heads, a.ncol), dim3(64), 0, s, a);
        else launch_combine<MC + 1>(a, nch, s);
    }
}
// nch: the chunk grid, the 64-key chunks of the launch's largest key count
void launch_attention(const AttnArgs& a, int nch, hipStream_t s) {
    if (nch < 1 || nch > ATT_MAX_CHUNKS || nch > a.max_chunks || a.ncol < 1 || a.ncol > MF_MAX_COLS)
        throw std::logic_error("internal: attention launch of " + std::to_string(nch) + " chunks over " +
                               std::to_string(a.ncol) + " columns (at most " + std::to_string(a.max_chunks) +
                               " chunk slots)");
    if (a.kv_cols) {
        // columns sharing caches (a prefill group's positions): each chunk is staged in LDS once
        // per ATT_PF_COLS query columns of its cache
        if (a.kv_cols > a.ncol) throw std::logic_error("internal: attention over more caches than columns");
        const int nq = (a.ncol + a.kv_cols - 1) / a.kv_cols, groups = (nq + ATT_PF_COLS - 1) / ATT_PF_COLS;
        // a 1-D grid: whole rows of 8 items (chunk, head, cache) times the query groups
        AttnArgs b = a;
        b.nch = nch;
        const int items = nch * a.heads * a.kv_cols;
        hipLaunchKernelGGL(k_attn_prefill, dim3((items + 7) / 8 * 8 * groups), dim3(64 * ATT_PF_WAVES), 0, s, b);
    } else {
        // one stream per column: K and V are read once per step (non-temporal)
        hipLaunchKernelGGL(k_attn_chunk, dim3(nch, a.heads, a.ncol), dim3(256), 0, s, a);
    }
    launch_combine<1>(a, nch, s);
}
// Sum over the 16 lanes of a lane group of 8 values per lane: levels 8, 4 and 2 halve the
// values, level 1 adds in place. Lanes t and t ^ 1 end with value 4*((t>>3)&1) + 2*((t>>2)&1) +
// ((t>>1)&1); each value's additions follow the butterfly p[l] + p[l+off], off = 8, 4, 2, 1.
__device__ __forceinline__ float halving8(const float (&p)[8], int t) {
    float a[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const bool lo = (t & 8) == 0;
        const float recv = xor_lane<8>(lo ? p[i + 4] : p[i]);
        a[i] = (lo ? p[i] : p[i + 4]) + recv;
    }
    float b[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const bool lo = (t & 4) == 0;
        const float recv = xor_lane<4>(lo ? a[i + 2] : a[i]);
        b[i] = (lo ? a[i] : a[i + 2]) + recv;
    }
    const bool lo = (t & 2) == 0;
    const float c = (lo ? b[0] : b[1]) + xor_lane<2>(lo ? b[1] : b[0]);
    return c + xor_lane<1>(c);
}

// The same cross-attention for n_ctx <= NK (one 64-key chunk; NK = 32 or 64 bounds the keys the
// wave loads and scores) by one wave per (head, request): the chunk of xattn_head with its
// combine reduced to out = fmaf(o, (float)(1 / sum), 0). One wave: head h of request r, of H
// heads and n_req requests.
template <int NK>
__device__ __forceinline__ void xattn_wave(const XAttnArgs& a, int h, int r, int H, int n_req) {
    static_assert(NK == 32 || NK == 64, "one wave scores 32 or 64 keys");
    constexpr int NIT = NK / 4, NMM = NK / 16;
    const int lane = threadIdx.x & 63, g = lane >> 4, t = lane & 15;
    const size_t kr = a.shared_kv ? 0 : (size_t)r;
    const float* K = a.k + (kr * H + h) * a.n_ctx * 64;
    const float* V = a.v + (kr * H + h) * a.n_ctx * 64;
    const float* bias = a.bias ? a.bias + ((size_t)h * n_req + r) * a.bias_stride : nullptr;
    __shared__ float el[64];
    __shared__ float4 ol[16];
    // every load first: q, the keys 4*it + g, the V rows g + 4k + 16mm, clamped to the n_ctx
    // rows the buffers hold (so no load waits for the request's own key count, read alongside;
    // rows past that count enter masked lanes only)
    const int rows = a.n_ctx;
    const float4 q = ((const float4*)(a.q + (size_t)r * a.dim + h * 64))[t];
    float4 kv[NIT], vv[4 * NMM];
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        const int j = it * 4 + g, jl = j < rows ? j : rows - 1;
        kv[it] = ((const float4*)(K + (size_t)jl * 64))[t];
    }
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int mm = 0; mm < NMM; ++mm) {
            const int j = g + 4 * k + 16 * mm, jl = j < rows ? j : rows - 1;
            vv[NMM * k + mm] = ((const float4*)(V + (size_t)jl * 64))[t];
        }
    const int nc = a.nc ? a.nc[r] : a.n_ctx;
    if (nc <= 0) {
        // no conditioning: zeros (the gated cross.out leaves the residual unchanged)
        put_act(a.out, r, h * 64 + lane, 0.0f, lane);
        if (a.out_f) a.out_f[(size_t)r * a.dim + h * 64 + lane] = 0.0f;
        return;
    }
    float p[NIT];
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        float v = __builtin_fmaf(q.x, kv[it].x, 0.0f);
        v = __builtin_fmaf(q.y, kv[it].y, v);
        v = __builtin_fmaf(q.z, kv[it].z, v);
        p[it] = __builtin_fmaf(q.w, kv[it].w, v);
    }
    // this lane's key after the halving reduce
    int jt;
    float sc;
    if constexpr (NK == 64) {
        jt = 4 * t + g;
        sc = halving16(p, t) * a.scale;
    } else {
        jt = 4 * (4 * ((t >> 3) & 1) + 2 * ((t >> 2) & 1) + ((t >> 1) & 1)) + g;
        sc = halving8(p, t) * a.scale;
    }
    if (bias && jt < nc) sc = sc + bias[jt];
    float m = jt < nc ? sc : -__builtin_inff();
    m = xor_reduce<32>(m, fmax_sel);
    if (NK == 64 || (t & 1) == 0) el[jt] = jt < nc ? dexpf(sc - m) : 0.0f;
    __syncthreads();
    const float f = (float)(1.0 / fold64d_b(lane < NK ? (double)el[lane] : 0.0));
    float4 P[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
        for (int mm = 0; mm < NMM; ++mm) {
            const int j = g + 4 * k + 16 * mm;
            acc = fmaf4_if(j < nc, el[j], vv[NMM * k + mm], acc);
        }
        P[k] = acc;
    }
    const float4 o4 = fold_partials16(P);
    if (lane < 16) ol[lane] = o4;
    __syncthreads();
    const float o = __builtin_fmaf(((const float*)ol)[lane], f, 0.0f);
    put_act(a.out, r, h * 64 + lane, o, lane);
    if (a.out_f) a.out_f[(size_t)r * a.dim + h * 64 + lane] = o;
}
template <int NK>
__global__ __launch_bounds__(64) void k_xattn_w(XAttnArgs a) {
    const unsigned long long t0 = stamp_begin(a.stamp);
    xattn_wave<NK>(a, blockIdx.x, blockIdx.y, gridDim.x, gridDim.y);
    stamp_end(a.stamp, t0);
}

void launch_xattn(const XAttnArgs& a, int heads, int n_req, hipStream_t s) {
    if (a.n_ctx <= 32) hipLaunchKernelGGL(k_xattn_w<32>, dim3(heads, n_req), dim3(64), 0, s, a);
    else if (a.n_ctx <= 64) hipLaunchKernelGGL(k_xattn_w<64>, dim3(heads, n_req), dim3(64), 0, s, a);
    else hipLaunchKernelGGL(k_xattn, dim3(heads, n_req), dim3(256), 0, s, a);
}
void launch_xkv_split(const float* kv, int n_ctx, int rows, int dim, float* k, float* v, hipStream_t s) {
    hipLaunchKernelGGL(k_xkv_split, dim3((n_ctx * 2 * dim + 255) / 256), dim3(256), 0, s, kv, n_ctx, rows, dim, k, v);
}
void launch_sample(const SampleArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(k_sample, dim3(a.n_q, a.n_req), dim3(256), 0, s, a);
}
__global__ void k_stamp_init(unsigned long long* p, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n * STAMP_SUB) { p[2 * i] = ~0ull; p[2 * i + 1] = 0ull; }
}
void launch_stamp_init(unsigned long long* p, int n, hipStream_t s) {
    hipLaunchKernelGGL(k_stamp_init, dim3((n * STAMP_SUB + 255) / 256), dim3(256), 0, s, p, n);
}
// Column preparation for a projection, one block per (column, role), the column built as the
// vector GEMV's prologue builds it (LayerNorm or the f32 column as is):
//  - role "quantize" (blockIdx.y == 0 when a.dst.q is set): the Q8 activation column, written
//    straight to a.dst (the matrix-core GEMV's source);
//  - role "A x" (the other blocks, when a.w.q is set; a.w = the adapter's A as an f32 matrix
//    [rank][in]): the inner mul_mat of lora.h:50-83's s * B(Ax). Wave w takes rank row
//    4 * (blockIdx.y - first) + w: lane l sums the 8-element units l, l + 64, ... of the row in
//    element order (fmaf), and the 64 partials fold by the butterfly -- the f32-weight
//    convention of every projection. Output a.y [col][a.y_stride].
template <int KG, bool LN>
__global__ __launch_bounds__(256) void k_prep(GemvArgs a) {
    extern __shared__ __align__(16) uint8_t lds[];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, col = blockIdx.x;
    const int in = a.w.in, nf = in / 4;
    double* red = (double*)(lds + (size_t)in * 4);
    float4 xr[KG], wr[KG], br[KG];
    const float4* xs = (const float4*)(a.x + (size_t)col * a.x_stride);
#pragma unroll
    for (int j = 0; j < KG; ++j) {
        const int f = tid + 256 * j < nf ? tid + 256 * j : nf - 1;
        xr[j] = xs[f];
        if (LN) { wr[j] = ((const float4*)a.ln_w)[f]; br[j] = ((const float4*)a.ln_b)[f]; }
    }
    const int first = a.dst.q ? 1 : 0;
    if ((int)blockIdx.y < first) {
        LdsAct g{};
        g.in = in;
        // F16 / F32 weights' activation form: the column's converted values, in place
        if (a.dst.kind == ACT_F16 || a.dst.kind == ACT_F32) {
            g.bm_col = -1;
            if (a.dst.kind == ACT_F16) {
                g.h = a.dst.h + (size_t)col * a.dst.stride;
                prologue<T_F16, KG, LN>(a, g, red, 0, tid, lane, xr, wr, br);
            } else {
                g.f = a.dst.f + (size_t)col * a.dst.stride;
                prologue<T_F32, KG, LN>(a, g, red, 0, tid, lane, xr, wr, br);
            }
            return;
        }
        g.bm_col = a.dst.bm ? col : -1;
        g.q = a.dst.bm ? a.dst.q : a.dst.q + (size_t)col * a.dst.stride;
        g.d = a.dst.bm ? a.dst.d : a.dst.d + (size_t)col * (a.dst.stride / 32);
        prologue<T_Q8_0, KG, LN>(a, g, red, 0, tid, lane, xr, wr, br);
        return;
    }
    LdsAct x{};
    x.in = in;
    x.bm_col = -1;
    x.f = (float*)lds;
    // this wave's row of A, read before the LayerNorm so it arrives during it (rows up to
    // 2048 wide: at most KA 8-element units per lane; wider rows read the rest afterwards)
    constexpr int KA = 4;
    const int k = ((int)blockIdx.y - first) * 4 + wave;
    const float* A = (const float*)a.w.q + (size_t)(k < a.w.out ? k : a.w.out - 1) * in;
    float4 wa[KA][2];
#pragma unroll
    for (int i = 0; i < KA; ++i) {
        const int u = lane + 64 * i, uc = u < in / 8 ? u : in / 8 - 1;
        wa[i][0] = *(const float4*)(A + 8 * uc);
        wa[i][1] = *(const float4*)(A + 8 * uc + 4);
    }
    prologue<T_F32, KG, LN>(a, x, red, 0, tid, lane, xr, wr, br);
    lds_barrier();
    if (k >= a.w.out) return;
    // units u = lane, lane + 64, ... in order: the prefetched ones, then any beyond
    const auto unit = [&](float p, const float4& w0, const float4& w1, int u) {
        const float4 x0 = *(const float4*)(x.f + 8 * u), x1 = *(const float4*)(x.f + 8 * u + 4);
        p = __builtin_fmaf(w0.x, x0.x, p); p = __builtin_fmaf(w0.y, x0.y, p);
        p = __builtin_fmaf(w0.z, x0.z, p); p = __builtin_fmaf(w0.w, x0.w, p);
        p = __builtin_fmaf(w1.x, x1.x, p); p = __builtin_fmaf(w1.y, x1.y, p);
        p = __builtin_fmaf(w1.z, x1.z, p); p = __builtin_fmaf(w1.w, x1.w, p);
        return p;
    };
    float p = 0.0f;
#pragma unroll
    for (int i = 0; i < KA; ++i)
        if (lane + 64 * i < in / 8) p = unit(p, wa[i][0], wa[i][1], lane + 64 * i);
    for (int u = lane + 64 * KA; u < in / 8; u += 64)
        p = unit(p, *(const float4*)(A + 8 * u), *(const float4*)(A + 8 * u + 4), u);
    p = fold64(p);
    if (lane == 0) a.y[(size_t)col * a.y_stride + k] = p;
}
template <int KG> static void prep_go(const GemvArgs& a, hipStream_t s) {
    const int ny = (a.dst.q ? 1 : 0) + (a.w.q ? (a.w.out + 3) / 4 : 0);
    const dim3 grid(a.ncol, ny);
    const size_t lds = (size_t)a.w.in * 4 + 512 * 8;
    if (a.pro == PRO_LN) hipLaunchKernelGGL((k_prep<KG, true>), grid, dim3(256), lds, s, a);
    else hipLaunchKernelGGL((k_prep<KG, false>), grid, dim3(256), lds, s, a);
}
static void prep_launch(const GemvArgs& a, hipStream_t s) {
    switch ((a.w.in + 1023) / 1024) {
    case 1: prep_go<1>(a, s); break;
    case 2: prep_go<2>(a, s); break;
    case 3: prep_go<3>(a, s); break;
    case 4: prep_go<4>(a, s); break;
    case 5: prep_go<5>(a, s); break;
    case 6: prep_go<6>(a, s); break;
    case 7: prep_go<7>(a, s); break;
    default: prep_go<8>(a, s); break;
    }
}
// A x of an f32 column (the f32 copy of an activation-form input), straight from global memory:
// one wave per (column, rank row); lane l sums the 8-element units l, l + 64, ... in element
// order (fmaf) -- NU of them, all loaded before the first product -- and the 64 partials fold
// by the butterfly: the same values k_prep's "A x" role computes from its LDS copy.
template <int NU>
__global__ __launch_bounds__(64) void k_ax_f32(GemvArgs a) {
    const int col = blockIdx.x, k = blockIdx.y, lane = threadIdx.x, units = a.w.in / 8;
    const float* A = (const float*)a.w.q + (size_t)k * a.w.in;
    const float* x = a.x + (size_t)col * a.x_stride;
    float4 w0[NU], w1[NU], x0[NU], x1[NU];
#pragma unroll
    for (int i = 0; i < NU; ++i) {
        const int u0 = lane + 64 * i, u = u0 < units ? u0 : units - 1;
        w0[i] = *(const float4*)(A + 8 * u); w1[i] = *(const float4*)(A + 8 * u + 4);
        x0[i] = *(const float4*)(x + 8 * u); x1[i] = *(const float4*)(x + 8 * u + 4);
    }
    __builtin_amdgcn_sched_barrier(0);   // every load in flight before the first product
    float p = 0.0f;
#pragma unroll
    for (int i = 0; i < NU; ++i) {
        if (lane + 64 * i >= units) break;
        p = __builtin_fmaf(w0[i].x, x0[i].x, p); p = __builtin_fmaf(w0[i].y, x0[i].y, p);
        p = __builtin_fmaf(w0[i].z, x0[i].z, p); p = __builtin_fmaf(w0[i].w, x0[i].w, p);
        p = __builtin_fmaf(w1[i].x, x1[i].x, p); p = __builtin_fmaf(w1[i].y, x1[i].y, p);
        p = __builtin_fmaf(w1[i].z, x1[i].z, p); p = __builtin_fmaf(w1[i].w, x1[i].w, p);
    }
    p = fold64(p);
    if (lane == 0) a.y[(size_t)col * a.y_stride + k] = p;
}
void launch_adapter_ax(const GemvArgs& a0, hipStream_t s) {
    GemvArgs a = a0;
    a.dst = ActBuf{};
    if (a.pro != PRO_F32) { prep_launch(a, s); return; }
    const dim3 grid(a.ncol, a.w.out);
    const int nu = (a.w.in / 8 + 63) / 64;
    if (nu <= 1) hipLaunchKernelGGL(k_ax_f32<1>, grid, dim3(64), 0, s, a);
    else if (nu <= 2) hipLaunchKernelGGL(k_ax_f32<2>, grid, dim3(64), 0, s, a);
    else if (nu <= 4) hipLaunchKernelGGL(k_ax_f32<4>, grid, dim3(64), 0, s, a);
    else if (nu <= 8) hipLaunchKernelGGL(k_ax_f32<8>, grid, dim3(64), 0, s, a);
    else if (nu <= 12) hipLaunchKernelGGL(k_ax_f32<12>, grid, dim3(64), 0, s, a);
    else hipLaunchKernelGGL(k_ax_f32<16>, grid, dim3(64), 0, s, a);
}
void launch_act_prep(const GemvArgs& a, hipStream_t s) { prep_launch(a, s); }

// Q8_0 scales tile-transposed: dt[(r/16 * nb + b) * 16 + r%16] = d[r * nb + b].
__global__ void k_scales_t(const uint16_t* d, int nb, int out, uint16_t* dt) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= out * nb) return;
    const int r = i / nb, b = i - r * nb;
    dt[((size_t)(r >> 4) * nb + b) * 16 + (r & 15)] = d[i];
}
// Q8_0 quants in operand order: qm[((r/16 * nb + b) * 64 + 16g + r%16) * 8 + j] = q[r][32b + 8g + j]
__global__ void k_weights_mf(const int8_t* q, int in, int out, int8_t* qm) {
    const size_t u = (size_t)blockIdx.x * 256 + threadIdx.x;   // one 8-byte piece
    const int nb = in / 32;
    if (u >= (size_t)out * nb * 4) return;
    const int lanei = (int)(u & 63);
    const size_t tb = u >> 6;
    const int b = (int)(tb % nb), tile = (int)(tb / nb);
    const int g = lanei >> 4, c = lanei & 15;
    *(uint2*)(qm + u * 8) = *(const uint2*)(q + (size_t)(tile * 16 + c) * in + b * 32 + 8 * g);
}
void launch_weights_mf(const DevMat& w, int8_t* qm, hipStream_t s) {
    const size_t n = (size_t)w.out * (w.in / 32) * 4;
    hipLaunchKernelGGL(k_weights_mf, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, (const int8_t*)w.q, w.in, w.out, qm);
}
// Q4_0 quants in operand order, one word per lane and block: byte m of lane (16g + r%16)'s word
// holds element 8g + m of row r's block (low nibble) and element 8g + m + 4 (high nibble); the
// device layout keeps ggml's block bytes (byte j: element j low, element j + 16 high).
__global__ void k_weights_mf4(const uint8_t* qs, int in, int out, uint32_t* qm) {
    const size_t u = (size_t)blockIdx.x * 256 + threadIdx.x;   // one 4-byte word
    const int nb = in / 32;
    if (u >= (size_t)out * nb * 4) return;
    const int lanei = (int)(u & 63);
    const size_t tb = u >> 6;
    const int b = (int)(tb % nb), tile = (int)(tb / nb);
    const int g = lanei >> 4, c = lanei & 15;
    const uint8_t* blk = qs + (size_t)(tile * 16 + c) * (in / 2) + b * 16;
    const auto nib = [&](int e) { return e < 16 ? (blk[e] & 15u) : (blk[e - 16] >> 4); };
    uint32_t w = 0;
    for (int m = 0; m < 4; ++m) w |= (nib(8 * g + m) | (nib(8 * g + m + 4) << 4)) << (8 * m);
    qm[u] = w;
}
void launch_weights_mf4(const DevMat& w, uint32_t* qm, hipStream_t s) {
    const size_t n = (size_t)w.out * (w.in / 32) * 4;
    hipLaunchKernelGGL(k_weights_mf4, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, (const uint8_t*)w.q, w.in,
                       w.out, qm);
}
void launch_scales_t(const DevMat& w, uint16_t* dt, hipStream_t s) {
    const int nb = w.in / 32;
    hipLaunchKernelGGL(k_scales_t, dim3((w.out * nb + 255) / 256), dim3(256), 0, s, w.d, nb, w.out, dt);
}

// DoRA rows (lora.h:11-32): one block per row. The block computes the row's dequantized weights
// and (BA)_i = (float) sum_k B[r][k] A[k][i] (double, k in order) for a segment of the row into
// LDS; thread 0 then adds the segment to the three double sums, each in increasing i.
constexpr int DORA_SEG = 2048;
__global__ __launch_bounds__(64) void k_dora_norm(DevMat w, const float* A, const float* B, int rank, float scale,
                                                  float* norm, int* bad) {
    __shared__ float wv[DORA_SEG], bav[DORA_SEG];
    const int r = blockIdx.x, tid = threadIdx.x, in = w.in;
    double sum = (double)in * 1e-12, t2 = 0.0, t3 = 0.0;
    int nonfinite = 0;
    for (int i0 = 0; i0 < in; i0 += DORA_SEG) {
        const int n = in - i0 < DORA_SEG ? in - i0 : DORA_SEG;
        for (int j = tid; j < n; j += 64) {
            double acc = 0.0;
            for (int k = 0; k < rank; ++k) acc += (double)B[(size_t)r * rank + k] * A[(size_t)k * in + i0 + j];
            bav[j] = (float)acc;
            const float x = mat_elem(w, r, i0 + j);
            nonfinite |= !__builtin_isfinite(x);
            wv[j] = x;
        }
        __syncthreads();
        if (tid == 0) {
            for (int j = 0; j < n; ++j) {
                const float x = wv[j], ba = bav[j];
                sum += (double)x * x;
                t2 += (double)x * ba;
                t3 += (double)ba * ba;
            }
        }
        __syncthreads();
    }
    if (tid == 0) {
        const float base = (float)sum;
        const double nsq = (double)base + 2.0 * scale * t2 + (double)scale * scale * t3;
        norm[r] = (float)__builtin_sqrt(nsq);
    }
    if (nonfinite) atomicOr(bad, 1);
}
void launch_dora_norm(const DevMat& w, const float* A, const float* B, int rank, float scale, float* norm, int* bad,
                      hipStream_t s) {
    hipLaunchKernelGGL(k_dora_norm, dim3(w.out), dim3(64), 0, s, w, A, B, rank, scale, norm, bad);
}
void launch_repack(int type, const uint8_t* raw, int64_t rows, int in, void* q, uint16_t* d, hipStream_t s) {
    const int64_t nblocks = rows * (in / 32);
    hipLaunchKernelGGL(k_repack, dim3((unsigned)((nblocks + 255) / 256)), dim3(256), 0, s, type, raw, nblocks, (int8_t*)q, d);
}

// ------------------------------------------------------------------------------------
// T5 encoder pieces (src/ac/t5.h:85-140)
// ------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_rows(DevMat m, const int32_t* ids, int n, float* out) {
    const int i = blockIdx.x * 256 + threadIdx.x, t = blockIdx.y;
    if (i >= m.in || t >= n) return;
    out[(size_t)t * m.in + i] = mat_elem(m, ids[t], i);
}
void launch_rows(const DevMat& m, const int32_t* ids, int n, float* out, hipStream_t s) {
    hipLaunchKernelGGL(k_rows, dim3((m.in + 255) / 256, n), dim3(256), 0, s, m, ids, n, out);
}

// One column per 256-thread block. Thread i owns partial i: float4 groups i, i+256, ... of the
// column, x*x (f32) summed in element order in double; the 256 partials folded by the butterfly
// (the same order as the LayerNorm prologue's sums).
__global__ __launch_bounds__(256) void k_rms(const float* x, int n, int stride, const float* w, float eps, float* y) {
    __shared__ double red[256];
    const int tid = threadIdx.x, lane = tid & 63, col = blockIdx.x, nf = n / 4;
    const float4* xs = (const float4*)(x + (size_t)col * stride);
    double acc = 0.0;
    for (int f = tid; f < nf; f += 256) {
        const float4 v = xs[f];
        acc = acc + (double)(v.x * v.x); acc = acc + (double)(v.y * v.y);
        acc = acc + (double)(v.z * v.z); acc = acc + (double)(v.w * v.w);
    }
    red[tid] = acc;
    __syncthreads();
    const float mean = (float)(fold256(red, lane) / (double)n);
    const float scale = 1.0f / __builtin_sqrtf(mean + eps);
    const float4* ws = (const float4*)w;
    float4* ys = (float4*)(y + (size_t)col * stride);
    for (int f = tid; f < nf; f += 256) {
        const float4 v = xs[f], g = ws[f];
        float4 o;
        o.x = v.x * scale; o.y = v.y * scale; o.z = v.z * scale; o.w = v.w * scale;
        o.x = o.x * g.x; o.y = o.y * g.y; o.z = o.z * g.z; o.w = o.w * g.w;
        ys[f] = o;
    }
}
void launch_rms(const float* x, int n, int ncol, int stride, const float* w, float eps, float* y, hipStream_t s) {
    hipLaunchKernelGGL(k_rms, dim3(ncol), dim3(256), 0, s, x, n, stride, w, eps, y);
}

// bias[h][query][key] = table[bucket(key - query)][h]; rel[r] holds the bucket of relative
// position r - zero.
__global__ __launch_bounds__(256) void k_t5_bias(DevMat table, const int32_t* rel, int zero, int seq, int heads,
                                                 float* bias) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= seq * seq * heads) return;
    const int h = i / (seq * seq), qk = i - h * seq * seq, qi = qk / seq, ki = qk - qi * seq;
    bias[i] = mat_elem(table, rel[ki - qi + zero], h) + 0.0f;
}
void launch_t5_bias(const DevMat& table, const int32_t* rel, int zero, int seq, int heads, float* bias, hipStream_t s) {
    hipLaunchKernelGGL(k_t5_bias, dim3((seq * seq * heads + 255) / 256), dim3(256), 0, s, table, rel, zero, seq, heads,
                       bias);
}

// n is a multiple of 32, so each 32-element block is one half-wave (the Q8 form's scale group).
__global__ __launch_bounds__(256) void k_relu_act(const float* x, int n, ActBuf dst) {
    const int i = blockIdx.x * 256 + threadIdx.x, col = blockIdx.y;
    if (i >= n) return;
    const float v = x[(size_t)col * n + i];
    put_act(dst, col, i, v > 0.0f ? v : 0.0f, threadIdx.x & 63);
}
void launch_relu_act(const float* x, int n, int ncol, const ActBuf& dst, hipStream_t s) {
    hipLaunchKernelGGL(k_relu_act, dim3((n + 255) / 256, ncol), dim3(256), 0, s, x, n, dst);
}

}  // namespace mgx
