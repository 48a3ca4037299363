// codec_kernels.h -- device kernels of the EnCodec / SEANet decoder (codec_kernels.hip).
// Layouts: features channel-major [C][T] (ggml [T, C]); conv weights [out][in][k]; transposed
// conv weights [out * k][in] (row o * k + j); LSTM matrices [4H][H].
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

namespace mgx {

// StreamableConv1d at stride 1 (src/ac/seanet.h:175-201): y[o][t] = b[o] + sum_i sum_j
// w[o][i][j] * act(x[i][reflect(t + j * dil - pad_left)]) (+ skip[o][t]); act is ELU when elu.
struct ConvArgs {
    const float* x;
    int cin, T;
    const float* w;
    const float* b;
    int cout, k, dil, pad_left, elu;
    const float* skip;   // optional residual [cout][T]
    float* y;
};
void launch_conv1d(const ConvArgs& a, hipStream_t s);

// StreamableConvTranspose1d (seanet.h:206-230): y[o][t] = b[o] + sum over taps j with
// (t + pad_left - j) a multiple of stride of w[o * k + j][i] * act(x[i][(t + pad_left - j) / stride]).
struct ConvTArgs {
    const float* x;
    int cin, T;
    const float* w;
    const float* b;
    int cout, k, stride, pad_left, elu;
    float* y;            // [cout][T * stride]
};
void launch_conv_transpose1d(const ConvTArgs& a, hipStream_t s);

// One LSTM time step (src/ac/lstm.h:60-96): g = proj[:, t] + w_hh h_prev; gates i, f, g, o;
// c = f * c + i * g; h = o * tanh(c). Writes h_next and out[:, t] (+ skip[:, t] when set).
struct LstmStepArgs {
    const float* w_hh;   // [4H][H]
    const float* proj;   // [4H][T]
    int H, T, t;
    const float* h_prev;
    float* h_next;
    float* c;
    float* out;          // [H][T]
    const float* skip;   // optional [H][T]
};
void launch_lstm_step(const LstmStepArgs& a, hipStream_t s);

// rvq_decode (src/mg/encodec.h:69-84): latent[d][t] = sum over levels, in order, of
// embed[level][codes[level][t]][d]. embed [n_q][bins][dim].
void launch_rvq_decode(const float* embed, const int32_t* codes, int n_q, int bins, int dim, int frames,
                       float* latent, hipStream_t s);

}  // namespace mgx
