"""The T5 encoder's host pieces through the C ABI, without a GPU: the relative-position bucket
(t5.h:46-61) against the reference's known-answer table (tests/t5_bucket_test.cpp) and
T5EncoderConfig::from (t5.h:31-43) on a GGUF file written by mgx.gguf."""
import json
import os

import pytest

import mgx
from mgx import gguf as G

HERE = os.path.dirname(os.path.abspath(__file__))


def test_library_bucket_matches_reference_table():
    d = json.load(open(os.path.join(HERE, "golden", "t5_bucket_cases.json")))
    for case in d["cases"]:
        assert mgx.t5_relative_bucket(case["relative_position"], d["num_buckets"], d["max_distance"]) == case["bucket"]
    for rp in range(-300, 301):
        b = mgx.t5_relative_bucket(rp)
        assert 0 <= b < 32 and (b >= 16) == (rp > 0)


def test_t5_config_from_gguf(tmp_path):
    m = mgx.SyntheticT5("t5-tiny", 1, seed=2)
    p = tmp_path / "t5.gguf"
    G.write_t5(str(p), m)
    g = mgx.Gguf(p)
    c = g.t5_config()
    for f, _ in mgx.T5Config._fields_:
        assert getattr(c, f) == getattr(m.config, f), f
    assert g.string("general.architecture") == "ac-t5"
    names = [t[0] for t in g.tensors()]
    assert names[:3] == ["te.embed.weight", "te.relative_attention_bias.weight", "te.0.attn_norm.weight"]
    g.close()
    kv = [e for e in G.t5_kv(m.config) if e[0] != "ac.t5.relative_buckets"]
    G.write_t5(str(p), m, kv=kv)
    with pytest.raises(mgx.MgxError, match="missing key: ac.t5.relative_buckets"):
        mgx.Gguf(p).t5_config()
