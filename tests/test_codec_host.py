"""The codec's host pieces through the C ABI, without a GPU: SeanetConfig::from
(src/ac/seanet.h:60-92) on GGUF files written by mgx.gguf, with the reference's messages."""
import pytest

import mgx
from mgx import gguf as G


def test_codec_config_from_gguf(tmp_path):
    m = mgx.SyntheticCodec("encodec-32k", seed=1)
    p = tmp_path / "codec.gguf"
    G.write_codec(str(p), m)
    c = mgx.Gguf(p).codec_config()
    want = mgx.CodecConfig.of(m.config)
    for f, _ in mgx.CodecConfig._fields_:
        if f != "ratios":
            assert getattr(c, f) == getattr(want, f), f
    assert list(c.ratios[:c.n_ratios]) == [8, 5, 4, 4] and c.hop_length == 640 and c.elu == 1 and c.rvq == 1


def test_codec_config_checks(tmp_path):
    m = mgx.SyntheticCodec("codec-tiny", seed=1)
    kv = G.codec_kv(m.config)
    p = tmp_path / "c.gguf"

    def expect(kv_, text):
        G.write_codec(str(p), m, kv=kv_)
        with pytest.raises(mgx.MgxError, match=text):
            mgx.Gguf(p).codec_config()

    expect([e if e[0] != "ac.codec.hop_length" else (e[0], G.U32, 7) for e in kv],
           "codec ratio product disagrees with the declared hop length")
    expect([e if e[0] != "ac.codec.ratios" else (e[0], G.ARR, (G.I32, [])) for e in kv], "codec has no ratios")
    expect([e for e in kv if e[0] != "ac.codec.lstm_layers"], "missing key: ac.codec.lstm_layers")
    expect([e if e[0] != "ac.architecture" else (e[0], G.STR, "x") for e in kv], "not an audiocraft GGUF")
