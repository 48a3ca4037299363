"""TEST INFRASTRUCTURE: a float64 numpy restatement of audiocraft.cpp's EnCodec decode path, the
checker for the library's codec decoder. Only tests/ and bench.py's cpu_baseline leg use it.

What it restates (reference file:line):
  conv geometry ............ src/ac/seanet.h:117-128 (StreamableConv1d padding)
  transposed geometry ...... src/ac/seanet.h:140-148 (StreamableConvTranspose1d trim)
  seanet_conv1d ............ src/ac/seanet.h:175-201 (reflect pad incl. the extra tail, conv, bias)
  seanet_conv_transpose1d .. src/ac/seanet.h:206-230 (columns = W x, col2im, trim, bias)
  seanet_residual .......... src/ac/seanet.h:234-242 (act, conv k, act, conv 1, identity skip)
  seanet_decode_pre/post ... src/ac/seanet.h:282-317
  lstm_graph ............... src/ac/lstm.h:44-101 (fused bias, gates i f g o, residual skip)
  rvq_decode ............... src/mg/encodec.h:69-84 (one lookup per level, summed in level order)
ELU is ggml_elu: x for x > 0, exp(x) - 1 otherwise. Everything is computed in float64; the
reference computes in f32 (ggml CPU), so a comparison against either is within f32 rounding.

Layouts: audio and features channel-major [C][T] (ggml [T, C]); conv weights torch order
[out][in][k] (ggml [k, in, out]); transposed-conv weights [out * k][in] with row o * k + j
(the converter's col2im layout, tools/convert_seanet.py:69-73); LSTM matrices [4H][H]; codebooks
[bins][dim]."""
import numpy as np


def ceil_div(a, b):
    return -(-a // b)


def conv_geometry(frames, kernel, stride, dilation):
    """(pad_left, pad_right, extra, out_frames)."""
    effective = (kernel - 1) * dilation + 1
    total = effective - stride
    extra = ceil_div(frames, stride) * stride - frames
    right = total // 2
    return total - right, right, extra, ceil_div(frames, stride)


def transpose_geometry(frames, kernel, stride):
    """(pad_left, pad_right, out_frames): the full transposed output is trimmed by pad_left on
    the left and pad_right on the right."""
    total = kernel - stride
    right = total // 2
    return total - right, right, frames * stride


def elu(x):
    return np.where(x > 0, x, np.expm1(np.minimum(x, 0.0)))


def conv1d(x, w, b, stride=1, dilation=1):
    """x [Cin][T], w [Cout][Cin][K], b [Cout] -> [Cout][ceil(T / stride)]."""
    x = np.asarray(x, np.float64)
    w = np.asarray(w, np.float64)
    cout, cin, k = w.shape
    frames = x.shape[1]
    left, right, extra, out = conv_geometry(frames, k, stride, dilation)
    if left or right + extra:
        if frames <= max(left, right + extra):
            raise ValueError("input too short for the reflect padding")
        x = np.pad(x, ((0, 0), (left, right + extra)), mode="reflect")
    y = np.zeros((cout, out))
    for j in range(k):
        start = j * dilation
        y += w[:, :, j] @ x[:, start:start + stride * (out - 1) + 1:stride]
    return y + np.asarray(b, np.float64)[:, None]


def conv_transpose1d(x, w_col2im, b, stride, out_channels):
    """x [Cin][T], w_col2im [out * k][Cin] -> [out][T * stride]."""
    x = np.asarray(x, np.float64)
    w = np.asarray(w_col2im, np.float64)
    k = w.shape[0] // out_channels
    frames = x.shape[1]
    left, right, out = transpose_geometry(frames, k, stride)
    cols = (w @ x).reshape(out_channels, k, frames)          # [o][j][t]
    full = np.zeros((out_channels, (frames - 1) * stride + k))
    for j in range(k):
        full[:, j:j + stride * (frames - 1) + 1:stride] += cols[:, j, :]
    return full[:, left:left + out] + np.asarray(b, np.float64)[:, None]


def sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def lstm(x, layers):
    """x [H][T]; layers: list of (w_ih [4H][H], w_hh [4H][H], bias [4H]). Returns the stack's
    output plus x (StreamableLSTM's skip)."""
    x = np.asarray(x, np.float64)
    H, T = x.shape
    inp = x
    for w_ih, w_hh, bias in layers:
        proj = np.asarray(w_ih, np.float64) @ inp + np.asarray(bias, np.float64)[:, None]
        w_hh = np.asarray(w_hh, np.float64)
        h = np.zeros(H)
        c = np.zeros(H)
        out = np.zeros((H, T))
        for t in range(T):
            g = proj[:, t] + w_hh @ h
            i, f, gg, o = sigmoid(g[:H]), sigmoid(g[H:2 * H]), np.tanh(g[2 * H:3 * H]), sigmoid(g[3 * H:])
            c = f * c + i * gg
            h = o * np.tanh(c)
            out[:, t] = h
        inp = out
    return inp + x


def rvq_decode(codes, embeds):
    """codes [n_q][frames], embeds: list of [bins][dim] -> latent [dim][frames]."""
    codes = np.asarray(codes)
    dim = embeds[0].shape[1]
    latent = np.zeros((dim, codes.shape[1]))
    for level, e in enumerate(embeds):
        latent += np.asarray(e, np.float64)[codes[level]].T
    return latent


def decoder_layout(cfg):
    """(stage, ratio, in_channels, out_channels, residual dilations) for each decoder stage."""
    mult = 2 ** len(cfg["ratios"])
    stages = []
    for s, ratio in enumerate(cfg["ratios"]):
        cin = cfg["n_filters"] * mult
        stages.append((s, ratio, cin, cin // 2, [cfg["dilation_base"] ** j for j in range(cfg["n_residual_layers"])]))
        mult //= 2
    return stages


def seanet_decode(cfg, W, latent):
    """latent [latent_dim][frames] -> audio [channels][frames * hop] (ELU codecs)."""
    x = conv1d(latent, W["codec.decoder.in.weight"], W["codec.decoder.in.bias"])
    x = lstm(x, [(W[f"codec.decoder.lstm.{l}.w_ih"], W[f"codec.decoder.lstm.{l}.w_hh"],
                  W[f"codec.decoder.lstm.{l}.bias"]) for l in range(cfg["lstm_layers"])])
    for s, ratio, cin, cout, dilations in decoder_layout(cfg):
        p = f"codec.decoder.stage.{s}."
        x = conv_transpose1d(elu(x), W[p + "up.weight_col2im"], W[p + "up.bias"], ratio, cout)
        for j, d in enumerate(dilations):
            r = p + f"res.{j}."
            h = conv1d(elu(x), W[r + "conv1.weight"], W[r + "conv1.bias"], 1, d)
            h = conv1d(elu(h), W[r + "conv2.weight"], W[r + "conv2.bias"])
            x = x + h
    return conv1d(elu(x), W["codec.decoder.out.weight"], W["codec.decoder.out.bias"])


def decode_codes(cfg, W, codes):
    embeds = [W[f"codec.rvq.{i}.embed"] for i in range(cfg["rvq_n_q"])]
    return seanet_decode(cfg, W, rvq_decode(codes, embeds))
