// codec_kernels.hip -- EnCodec / SEANet decoder kernels for gfx950 (declared in codec_kernels.h).
//
// The decoder is f32 convolution over long sequences (30 s of 32 kHz audio is 960000 samples
// through 64 channels in the last stage). A block computes a 32-channel x 128-sample output tile
// (8 x 32 threads, each 4 channels x 4 samples, the 4 samples 32 apart so a wave's loads and
// stores are contiguous); input channels are staged 8 at a time through LDS with the reflect
// padding, and ELU, applied on the way in. The LSTM runs one launch per time step: its 16 MB
// recurrent matrix (H = 1024) stays in the last-level cache between steps.
#include "codec_kernels.h"

namespace mgx {

namespace {

constexpr int TT = 128;   // output samples per block
constexpr int ICT = 8;    // input channels per LDS stage

__device__ __forceinline__ float elu_f(float v) { return v > 0.0f ? v : expm1f(v); }
__device__ __forceinline__ float sigmoid_f(float v) { return 1.0f / (1.0f + expf(-v)); }

template <int CPT>
__global__ __launch_bounds__(256) void k_conv1d(ConvArgs a) {
    constexpr int OCT = 8 * CPT;
    extern __shared__ float lds[];
    const int W = TT + (a.k - 1) * a.dil;
    float* xs = lds;               // [ICT][W]
    float* ws = lds + ICT * W;     // [OCT][ICT][k]
    const int tid = threadIdx.x, tx = tid & 31, ty = tid >> 5;
    const int t0 = blockIdx.x * TT, o0 = blockIdx.y * OCT;
    float acc[CPT][4];
#pragma unroll
    for (int c = 0; c < CPT; ++c)
#pragma unroll
        for (int m = 0; m < 4; ++m) acc[c][m] = 0.0f;
    for (int i0 = 0; i0 < a.cin; i0 += ICT) {
        for (int idx = tid; idx < ICT * W; idx += 256) {
            const int i = idx / W, u = idx - i * W;
            // reflect once (the host checks both pads are shorter than T); positions that
            // only feed samples past T are clamped into range
            int tt = t0 + u - a.pad_left;
            tt = tt < 0 ? -tt : tt;
            tt = tt >= a.T ? 2 * (a.T - 1) - tt : tt;
            tt = tt < 0 ? 0 : tt;
            float v = 0.0f;
            if (i0 + i < a.cin) {
                v = a.x[(size_t)(i0 + i) * a.T + tt];
                if (a.elu) v = elu_f(v);
            }
            xs[idx] = v;
        }
        for (int idx = tid; idx < OCT * ICT * a.k; idx += 256) {
            const int oo = idx / (ICT * a.k), rem = idx - oo * ICT * a.k, i = rem / a.k, j = rem - i * a.k;
            ws[idx] = (o0 + oo < a.cout && i0 + i < a.cin) ? a.w[((size_t)(o0 + oo) * a.cin + i0 + i) * a.k + j] : 0.0f;
        }
        __syncthreads();
        for (int i = 0; i < ICT; ++i)
            for (int j = 0; j < a.k; ++j) {
                float xv[4];
#pragma unroll
                for (int m = 0; m < 4; ++m) xv[m] = xs[i * W + tx + 32 * m + j * a.dil];
#pragma unroll
                for (int c = 0; c < CPT; ++c) {
                    const float wv = ws[((ty * CPT + c) * ICT + i) * a.k + j];
#pragma unroll
                    for (int m = 0; m < 4; ++m) acc[c][m] = __builtin_fmaf(wv, xv[m], acc[c][m]);
                }
            }
        __syncthreads();
    }
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
        const int o = o0 + ty * CPT + c;
        if (o >= a.cout) continue;
        const float bo = a.b[o];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const int t = t0 + tx + 32 * m;
            if (t >= a.T) continue;
            float v = acc[c][m] + bo;
            if (a.skip) v = a.skip[(size_t)o * a.T + t] + v;
            a.y[(size_t)o * a.T + t] = v;
        }
    }
}

// The input window of a 128-sample output tile: indices jlo .. jlo + W - 1 with
// jlo = (t0 + pad_left) / stride - (taps - 1).
template <int CPT>
__global__ __launch_bounds__(256) void k_conv_t(ConvTArgs a, int taps, int W) {
    constexpr int OCT = 8 * CPT;
    extern __shared__ float lds[];
    float* xs = lds;               // [ICT][W]
    float* ws = lds + ICT * W;     // [OCT][k][ICT]
    const int tid = threadIdx.x, tx = tid & 31, ty = tid >> 5;
    const int t0 = blockIdx.x * TT, o0 = blockIdx.y * OCT, s = a.stride, To = a.T * s;
    const int jlo = (t0 + a.pad_left) / s - (taps - 1);
    float acc[CPT][4];
#pragma unroll
    for (int c = 0; c < CPT; ++c)
#pragma unroll
        for (int m = 0; m < 4; ++m) acc[c][m] = 0.0f;
    for (int i0 = 0; i0 < a.cin; i0 += ICT) {
        for (int idx = tid; idx < ICT * W; idx += 256) {
            const int i = idx / W, u = idx - i * W, j = jlo + u;
            float v = 0.0f;
            if (i0 + i < a.cin && j >= 0 && j < a.T) {
                v = a.x[(size_t)(i0 + i) * a.T + j];
                if (a.elu) v = elu_f(v);
            }
            xs[idx] = v;
        }
        for (int idx = tid; idx < OCT * a.k * ICT; idx += 256) {
            const int oo = idx / (a.k * ICT), rem = idx - oo * a.k * ICT, jj = rem / ICT, i = rem - jj * ICT;
            ws[idx] = (o0 + oo < a.cout && i0 + i < a.cin) ? a.w[((size_t)(o0 + oo) * a.k + jj) * a.cin + i0 + i] : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const int q = t0 + tx + 32 * m + a.pad_left, jq = q / s, p = q - jq * s;
            for (int mm = 0; mm < taps; ++mm) {
                const int jj = p + mm * s;
                if (jj >= a.k) break;
                const float* xr = xs + (jq - mm - jlo);
                for (int i = 0; i < ICT; ++i) {
                    const float xv = xr[i * W];
#pragma unroll
                    for (int c = 0; c < CPT; ++c)
                        acc[c][m] = __builtin_fmaf(ws[((ty * CPT + c) * a.k + jj) * ICT + i], xv, acc[c][m]);
                }
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
        const int o = o0 + ty * CPT + c;
        if (o >= a.cout) continue;
        const float bo = a.b[o];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const int t = t0 + tx + 32 * m;
            if (t < To) a.y[(size_t)o * To + t] = acc[c][m] + bo;
        }
    }
}

// 8 hidden units per block: wave g computes gate g's 8 rows (lane-strided dot products,
// butterfly), then 8 threads update their unit's cell.
__global__ __launch_bounds__(256) void k_lstm_step(LstmStepArgs a) {
    extern __shared__ float hs[];
    __shared__ float gsum[32];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, j0 = blockIdx.x * 8, H = a.H;
    for (int e = tid; e < H; e += 256) hs[e] = a.h_prev[e];
    __syncthreads();
    for (int uu = 0; uu < 8; ++uu) {
        const int j = j0 + uu;
        float acc = 0.0f;
        if (j < H) {
            const float* row = a.w_hh + (size_t)(wave * H + j) * H;
            for (int e = lane; e < H; e += 64) acc = __builtin_fmaf(row[e], hs[e], acc);
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, 64);
        if (lane == 0 && j < H) gsum[wave * 8 + uu] = a.proj[(size_t)(wave * H + j) * a.T + a.t] + acc;
    }
    __syncthreads();
    if (tid < 8 && j0 + tid < H) {
        const int j = j0 + tid;
        const float ig = sigmoid_f(gsum[tid]), fg = sigmoid_f(gsum[8 + tid]);
        const float gg = tanhf(gsum[16 + tid]), og = sigmoid_f(gsum[24 + tid]);
        const float c = fg * a.c[j] + ig * gg;
        const float h = og * tanhf(c);
        a.c[j] = c;
        a.h_next[j] = h;
        a.out[(size_t)j * a.T + a.t] = a.skip ? h + a.skip[(size_t)j * a.T + a.t] : h;
    }
}

// The same step with one wave per hidden unit: the wave loads its unit's four gate rows as
// float4s, PER per lane per row (H = 256 * PER), every load issued before the first product;
// 4 units per block, H / 4 blocks.
template <int PER>
__global__ __launch_bounds__(256) void k_lstm_step_w(LstmStepArgs a) {
    extern __shared__ float hs[];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, H = a.H, j = blockIdx.x * 4 + wave;
    float4 wv[4][PER];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const float4* row = (const float4*)(a.w_hh + (size_t)(g * H + j) * H);
#pragma unroll
        for (int p = 0; p < PER; ++p) wv[g][p] = row[lane + 64 * p];
    }
    float pj[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) pj[g] = a.proj[(size_t)(g * H + j) * a.T + a.t];
    for (int e = tid; e < H; e += 256) hs[e] = a.h_prev[e];
    __syncthreads();
    const float4* h4 = (const float4*)hs;
    float acc[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        float v = 0.0f;
#pragma unroll
        for (int p = 0; p < PER; ++p) {
            const float4 h = h4[lane + 64 * p];
            v = __builtin_fmaf(wv[g][p].x, h.x, v);
            v = __builtin_fmaf(wv[g][p].y, h.y, v);
            v = __builtin_fmaf(wv[g][p].z, h.z, v);
            v = __builtin_fmaf(wv[g][p].w, h.w, v);
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
        acc[g] = v;
    }
    if (lane == 0) {
        const float ig = sigmoid_f(pj[0] + acc[0]), fg = sigmoid_f(pj[1] + acc[1]);
        const float gg = tanhf(pj[2] + acc[2]), og = sigmoid_f(pj[3] + acc[3]);
        const float c = fg * a.c[j] + ig * gg;
        const float h = og * tanhf(c);
        a.c[j] = c;
        a.h_next[j] = h;
        a.out[(size_t)j * a.T + a.t] = a.skip ? h + a.skip[(size_t)j * a.T + a.t] : h;
    }
}

__global__ __launch_bounds__(256) void k_rvq_decode(const float* embed, const int32_t* codes, int n_q, int bins,
                                                    int dim, int frames, float* latent) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= dim * frames) return;
    const int d = i / frames, t = i - d * frames;
    float v = 0.0f;
    for (int l = 0; l < n_q; ++l) v = v + embed[((size_t)l * bins + codes[(size_t)l * frames + t]) * dim + d];
    latent[i] = v;
}

}  // namespace

void launch_conv1d(const ConvArgs& a, hipStream_t s) {
    const int W = TT + (a.k - 1) * a.dil;
    if (a.cout >= 32) {
        const size_t lds = sizeof(float) * ((size_t)ICT * W + (size_t)32 * ICT * a.k);
        hipLaunchKernelGGL(k_conv1d<4>, dim3((a.T + TT - 1) / TT, (a.cout + 31) / 32), dim3(256), lds, s, a);
    } else {
        const size_t lds = sizeof(float) * ((size_t)ICT * W + (size_t)8 * ICT * a.k);
        hipLaunchKernelGGL(k_conv1d<1>, dim3((a.T + TT - 1) / TT, (a.cout + 7) / 8), dim3(256), lds, s, a);
    }
}

void launch_conv_transpose1d(const ConvTArgs& a, hipStream_t s) {
    const int taps = (a.k + a.stride - 1) / a.stride;
    const int W = (TT - 1) / a.stride + taps + 2;
    const int To = a.T * a.stride;
    if (a.cout >= 32) {
        const size_t lds = sizeof(float) * ((size_t)ICT * W + (size_t)32 * a.k * ICT);
        hipLaunchKernelGGL(k_conv_t<4>, dim3((To + TT - 1) / TT, (a.cout + 31) / 32), dim3(256), lds, s, a, taps, W);
    } else {
        const size_t lds = sizeof(float) * ((size_t)ICT * W + (size_t)8 * a.k * ICT);
        hipLaunchKernelGGL(k_conv_t<1>, dim3((To + TT - 1) / TT, (a.cout + 7) / 8), dim3(256), lds, s, a, taps, W);
    }
}

void launch_lstm_step(const LstmStepArgs& a, hipStream_t s) {
    const size_t lds = sizeof(float) * (size_t)a.H;
    switch (a.H % 256 ? 0 : a.H / 256) {
    case 1: hipLaunchKernelGGL(k_lstm_step_w<1>, dim3(a.H / 4), dim3(256), lds, s, a); break;
    case 2: hipLaunchKernelGGL(k_lstm_step_w<2>, dim3(a.H / 4), dim3(256), lds, s, a); break;
    case 4: hipLaunchKernelGGL(k_lstm_step_w<4>, dim3(a.H / 4), dim3(256), lds, s, a); break;
    case 8: hipLaunchKernelGGL(k_lstm_step_w<8>, dim3(a.H / 4), dim3(256), lds, s, a); break;
    default: hipLaunchKernelGGL(k_lstm_step, dim3((a.H + 7) / 8), dim3(256), lds, s, a); break;
    }
}

void launch_rvq_decode(const float* embed, const int32_t* codes, int n_q, int bins, int dim, int frames,
                       float* latent, hipStream_t s) {
    hipLaunchKernelGGL(k_rvq_decode, dim3((dim * frames + 255) / 256), dim3(256), 0, s, embed, codes, n_q, bins, dim,
                       frames, latent);
}

}  // namespace mgx
