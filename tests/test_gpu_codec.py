"""The EnCodec decoder (mgx_codec_*) on the GPU against the float64 oracle (oracle/codec_ref.py,
restating src/mg/encodec.h:69-84, src/ac/seanet.h:282-317, src/ac/lstm.h:44-101). Both compute
in f32 against a float64 restatement, so the check is a tolerance: the largest absolute error
over the decode is at most 1e-4 of the decode's peak amplitude (f32 rounding through the
conv stack and the LSTM recurrence stays near 1e-6)."""
import numpy as np
import pytest

from mgx import gguf as G
from mgx import synth
from oracle import codec_ref as K

pytestmark = pytest.mark.gpu
TOL = 1e-4


@pytest.fixture(scope="module")
def M():
    import mgx
    mgx.load()
    return mgx


def close(got, want, what):
    err = np.abs(got - want).max() / np.abs(want).max()
    print(f"{what}: relative max error {err:.2e}", flush=True)
    assert got.shape == want.shape and err <= TOL, f"{what}: {err}"


@pytest.mark.parametrize("shape,frames", [("codec-tiny", 4), ("codec-tiny", 20), ("codec-mini", 50),
                                          ("encodec-32k", 12)])
def test_decode_matches_oracle(M, shape, frames):
    print(f"codec decode {shape} frames={frames}", flush=True)
    m = synth.SyntheticCodec(shape, seed=frames)
    k = M.Codec(m.config, m.tensors)
    codes = m.codes(frames + 1, frames)
    close(k.decode(codes), K.decode_codes(m.config, m.weights, codes), f"{shape} {frames}")
    k.close()


def test_encodec_five_seconds(M):
    """EnCodec 32 kHz at its real widths over 250 frames (5 s, 160000 samples), then a short
    decode on the same codec (buffers grown once, reused)."""
    print("encodec-32k 250 frames", flush=True)
    m = synth.SyntheticCodec("encodec-32k", seed=5)
    k = M.Codec(m.config, m.tensors)
    codes = m.codes(6, 250)
    close(k.decode(codes), K.decode_codes(m.config, m.weights, codes), "encodec-32k 250")
    codes = m.codes(7, 9)
    close(k.decode(codes), K.decode_codes(m.config, m.weights, codes), "encodec-32k 9 after 250")
    k.close()


def test_decode_latent(M):
    m = synth.SyntheticCodec("codec-mini", seed=8)
    k = M.Codec(m.config, m.tensors)
    lat = np.random.default_rng(2).normal(0, 1, (m.config["latent_dim"], 30)).astype(np.float32)
    close(k.decode_latent(lat), K.seanet_decode(m.config, m.weights, lat), "latent")
    k.close()


def test_codec_from_gguf_and_checks(M, tmp_path):
    m = synth.SyntheticCodec("codec-tiny", seed=9)
    p = tmp_path / "codec.gguf"
    G.write_codec(str(p), m)
    g = M.Gguf(p)
    k = M.Codec.from_gguf(g)
    g.close()
    codes = m.codes(10, 16)
    close(k.decode(codes), K.decode_codes(m.config, m.weights, codes), "gguf")
    bad = codes.copy()
    bad[1, 3] = m.config["rvq_bins"]
    with pytest.raises(M.MgxError, match=r"a code is outside \[0, bins\)"):
        k.decode(bad)
    with pytest.raises(M.MgxError, match="too short"):
        k.decode(codes[:, :3])
    k.close()
    with pytest.raises(M.MgxError, match="codec.decoder.stage.1.up.bias"):
        M.Codec(m.config, [t for t in m.tensors if t[0] != "codec.decoder.stage.1.up.bias"])
    with pytest.raises(M.MgxError, match="only ELU codecs"):
        M.Codec(dict(m.config, activation="snake"), m.tensors)
