"""The codec oracle (oracle/codec_ref.py, restating src/ac/seanet.h, src/ac/lstm.h and
src/mg/encodec.h) pinned on the CPU: the LSTM against torch.nn.LSTM's vectors held by the
reference's tests/lstm_test.cpp, the residual quantizer's decode against transformers' vectors
in tests/codec_test.cpp, the padding arithmetic against the closed forms of
tests/seanet_shape_test.cpp, the convolutions against numpy's own convolution and the
transposed convolution against the adjoint identity <conv_T x, y> = <x, conv y>."""
import json
import os

import numpy as np
import pytest

from mgx import synth
from oracle import codec_ref as K

HERE = os.path.dirname(os.path.abspath(__file__))


def test_lstm_matches_torch_vectors():
    d = json.load(open(os.path.join(HERE, "golden", "lstm_cases.json")))
    H, T, L, a = d["hidden"], d["frames"], d["layers"], d["arrays"]
    layers = [(np.array(a[f"w_ih{l}"]).reshape(4 * H, H), np.array(a[f"w_hh{l}"]).reshape(4 * H, H),
               np.array(a[f"bias{l}"])) for l in range(L)]
    x = np.array(a["input_seq"]).reshape(T, H).T                 # [H][T]
    got = K.lstm(x, layers).T.reshape(-1)
    assert np.abs(got - np.array(a["expected"])).max() < 1e-6


def test_rvq_decode_matches_transformers_vectors():
    d = json.load(open(os.path.join(HERE, "golden", "rvq_cases.json")))
    nq, bins, dim, frames = d["n_q"], d["bins"], d["dim"], d["frames"]
    embeds = list(np.array(d["embed"]).reshape(nq, bins, dim))
    codes = np.array(d["codes"]).reshape(nq, frames)
    got = K.rvq_decode(codes, embeds)
    assert np.abs(got.reshape(-1) - np.array(d["quantized"])).max() < 1e-5


@pytest.mark.parametrize("frames,kernel,stride,dilation", [
    (960000, 7, 1, 1), (960000, 8, 4, 1), (60000, 10, 5, 1), (12000, 16, 8, 1), (1500, 3, 1, 2), (1500, 3, 1, 4),
    (1000, 4, 2, 1), (1001, 6, 3, 1), (1003, 10, 5, 1), (7, 12, 6, 1), (13, 16, 8, 1)])
def test_conv_geometry(frames, kernel, stride, dilation):
    """seanet_shape_test.cpp:26-60: audiocraft's get_extra_padding_for_conv1d and halves."""
    left, right, extra, out = K.conv_geometry(frames, kernel, stride, dilation)
    total = (kernel - 1) * dilation + 1 - stride
    n = (frames - ((kernel - 1) * dilation + 1) + total) / stride + 1
    ideal = (int(np.ceil(n)) - 1) * stride + ((kernel - 1) * dilation + 1) - total
    assert extra == ideal - frames and right == total // 2 and left + right == total
    assert out == -(-frames // stride)
    assert (frames + left + right + extra - ((kernel - 1) * dilation + 1)) // stride + 1 == out


@pytest.mark.parametrize("frames", [1, 2, 17, 750])
@pytest.mark.parametrize("stride", [2, 3, 4, 5, 6, 7, 8])
def test_transpose_geometry(frames, stride):
    left, right, out = K.transpose_geometry(frames, 2 * stride, stride)
    assert out == frames * stride and left - right == stride % 2 and left + right == stride


def test_conv1d_against_numpy_convolve():
    rng = np.random.default_rng(1)
    x = rng.normal(size=(1, 50))
    w = rng.normal(size=(1, 1, 7))
    got = K.conv1d(x, w, np.zeros(1))
    xp = np.pad(x[0], (3, 3), mode="reflect")
    want = np.convolve(xp, w[0, 0, ::-1], mode="valid")         # correlation = convolution with the flip
    assert np.abs(got[0] - want).max() < 1e-12
    # dilation 2, two channels in, three out
    x = rng.normal(size=(2, 40))
    w = rng.normal(size=(3, 2, 3))
    got = K.conv1d(x, w, np.arange(3.0), 1, 2)
    xp = np.pad(x, ((0, 0), (2, 2)), mode="reflect")
    for o in range(3):
        want = sum(np.convolve(xp[i], np.repeat(w[o, i, ::-1], 2)[:-1] * np.array([1, 0, 1, 0, 1]), mode="valid")
                   for i in range(2)) + o
        assert np.abs(got[o] - want).max() < 1e-12


@pytest.mark.parametrize("stride", [2, 3, 5])
def test_conv_transpose_is_the_adjoint(stride):
    """Without trimming, conv_transpose(x) . y == x . conv(y) for the same kernel (the
    definition of a transposed convolution); the oracle's trim is then checked separately."""
    rng = np.random.default_rng(stride)
    cin, cout, k, T = 3, 2, 2 * stride, 9
    w = rng.normal(size=(cin, cout, k))                            # torch ConvTranspose1d [in][out][k]
    x = rng.normal(size=(cin, T))
    wc = w.reshape(cin, cout * k).T                                 # the converter's col2im layout
    left, right, _ = K.transpose_geometry(T, k, stride)
    full_len = (T - 1) * stride + k
    y = rng.normal(size=(cout, full_len))
    got = K.conv_transpose1d(x, wc, np.zeros(cout), stride, cout)
    # rebuild the untrimmed output from the trimmed one plus the trimmed edges via the adjoint
    conv_y = np.zeros((cin, T))                                     # strided correlation, no padding
    for t in range(T):
        conv_y[:, t] = np.einsum("iok,ok->i", w, y[:, t * stride:t * stride + k])
    y_mid = np.zeros_like(y)
    y_mid[:, left:left + T * stride] = y[:, left:left + T * stride]
    conv_mid = np.zeros((cin, T))
    for t in range(T):
        conv_mid[:, t] = np.einsum("iok,ok->i", w, y_mid[:, t * stride:t * stride + k])
    assert abs((got * y[:, left:left + T * stride]).sum() - (x * conv_mid).sum()) < 1e-9
    assert got.shape == (cout, T * stride)


def test_seanet_decode_shapes_and_finite():
    m = synth.SyntheticCodec("codec-tiny", seed=3)
    c = m.config
    codes = m.codes(4, 20)
    audio = K.decode_codes(c, m.weights, codes)
    assert audio.shape == (1, 20 * c["hop_length"]) and np.isfinite(audio).all() and np.abs(audio).max() > 0
    # a planted mistake -- no ELU anywhere -- changes the audio well beyond f32 rounding
    elu = K.elu
    try:
        K.elu = lambda x: x
        wrong = K.decode_codes(c, m.weights, codes)
    finally:
        K.elu = elu
    assert np.abs(audio - wrong).max() > 1e-2
