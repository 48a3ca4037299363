"""The oracle's T5 encoder (oracle/cpu_ref.c ref_t5_*, restating src/ac/t5.h:46-140) pinned on the
CPU: the relative-position buckets against the reference's own known-answer table
(tests/t5_bucket_test.cpp, from transformers), RMS norm exactly against a float32 emulation, and
the whole encoder against an independent float64 formulation of T5 (t5.h:85-140 /
transformers' T5 encoder)."""
import json
import os

import numpy as np
import pytest

from mgx import synth
from oracle import cpu_ref as R

HERE = os.path.dirname(os.path.abspath(__file__))


def test_buckets_match_reference_table():
    d = json.load(open(os.path.join(HERE, "golden", "t5_bucket_cases.json")))
    assert len(d["cases"]) == 27
    for case in d["cases"]:
        got = R.t5_bucket(case["relative_position"], d["num_buckets"], d["max_distance"])
        assert got == case["bucket"], case


def test_bucket_properties():
    """In range, the sign split on the two halves, monotone in distance, 0 on the diagonal
    (t5_bucket_test.cpp:39-71 checks the first three)."""
    prev_pos, prev_neg = -1, -1
    for rp in range(0, 301):
        b = R.t5_bucket(rp)
        assert 0 <= b < 32 and (b >= 16) == (rp > 0)
        if rp > 0:
            assert b >= prev_pos
            prev_pos = b
        bn = R.t5_bucket(-rp)
        assert 0 <= bn < 16 and bn >= prev_neg
        prev_neg = bn
    assert R.t5_bucket(0) == 0
    # small distances map one to one (a quarter of the buckets each side)
    assert [R.t5_bucket(-i) for i in range(8)] == list(range(8))
    assert [R.t5_bucket(i) for i in range(1, 8)] == [16 + i for i in range(1, 8)]


def test_rms_norm_exact():
    """mean of squares in double (the float products are exact in double and their double sum
    does not depend on order for these ranges), scale = 1/sqrtf(mean + eps) in f32, then
    (x * scale) * w rounded twice -- bit for bit."""
    rng = np.random.default_rng(5)
    for n in (128, 768, 3072):
        x = rng.normal(0, 2.0, n).astype(np.float32)
        w = (1 + rng.normal(0, 0.1, n)).astype(np.float32)
        got = R.rms_norm(x, w, 1e-6)
        sq = (x * x).astype(np.float64).sum()
        mean = np.float32(sq / n)
        scale = np.float32(1.0) / np.sqrt(np.float32(mean + np.float32(1e-6)), dtype=np.float32)
        want = (x * scale).astype(np.float32) * w
        assert np.array_equal(got, want.astype(np.float32)), n
    # a planted mistake -- the mean subtracted as LayerNorm does -- is caught by the same check
    x = rng.normal(3.0, 1.0, 768).astype(np.float32)
    w = np.ones(768, np.float32)
    ln = (x - x.mean()) / np.sqrt(((x - x.mean()) ** 2).mean() + 1e-6)
    assert np.abs(R.rms_norm(x, w, 1e-6) - ln).max() > 0.5


def dense(t):
    """A ggml tensor (name, type, ne0, ne1, bytes) as float64 [ne1][ne0]."""
    name, ttype, ne0, ne1, data = t
    if ttype == 0:
        return data.view(np.float32).reshape(ne1, ne0).astype(np.float64)
    if ttype == 1:
        return data.view(np.float16).reshape(ne1, ne0).astype(np.float64)
    raise ValueError("F32 / F16 only here")


def t5_float64(c, tensors, ids):
    """T5-base's encoder in float64: embedding rows, per layer x += o(attn(rms(x))) with
    scores q.k (no 1/sqrt(d)) + bias[h][q][k] = table[bucket(k - q)][h], then x +=
    wo(relu(wi(rms(x)))); final rms."""
    W = {t[0]: dense(t) for t in tensors}
    H, hd = c.heads, c.head_dim
    seq = len(ids)

    def rms(x, w):
        return x / np.sqrt((x * x).mean(axis=1, keepdims=True) + c.eps) * w[0]

    x = W["te.embed.weight"][ids]
    table = W["te.relative_attention_bias.weight"]            # [buckets][heads]
    bucket = np.array([[R.t5_bucket(k - q, c.relative_buckets, c.relative_max_distance) for k in range(seq)]
                       for q in range(seq)])
    bias = table[bucket].transpose(2, 0, 1)                    # [h][q][k]
    for l in range(c.layers):
        p = f"te.{l}."
        h = rms(x, W[p + "attn_norm.weight"])
        q, k, v = (h @ W[p + n + ".weight"].T for n in ("q", "k", "v"))
        o = np.zeros_like(q)
        for hh in range(H):
            sl = slice(hh * hd, (hh + 1) * hd)
            s = q[:, sl] @ k[:, sl].T + bias[hh]
            s = np.exp(s - s.max(axis=1, keepdims=True))
            o[:, sl] = (s / s.sum(axis=1, keepdims=True)) @ v[:, sl]
        x = x + o @ W[p + "o.weight"].T
        h = rms(x, W[p + "ffn_norm.weight"])
        x = x + np.maximum(h @ W[p + "wi.weight"].T, 0.0) @ W[p + "wo.weight"].T
    return rms(x, W["te.norm.weight"])


@pytest.mark.parametrize("wtype,tol", [(0, 2e-5), (1, 5e-3)])
@pytest.mark.parametrize("seq", [1, 7, 40])
def test_encoder_against_float64(wtype, tol, seq):
    m = synth.SyntheticT5("t5-tiny", wtype, seed=3)
    ids = synth.synth_ids(seq, seq, m.config.vocab)
    got = R.t5_encode(m.config, m.tensors, ids)
    want = t5_float64(m.config, m.tensors, ids)
    err = np.abs(got - want).max() / np.abs(want).max()
    assert err < tol, err


def test_encoder_bias_orientation_matters():
    """The same check fails when the bias is transposed ([k][q]) -- the check can see it."""
    m = synth.SyntheticT5("t5-tiny", 0, seed=4)
    ids = synth.synth_ids(9, 12, m.config.vocab)
    got = R.t5_encode(m.config, m.tensors, ids)
    orig = R.t5_bucket
    try:
        R.t5_bucket = lambda rp, nb=32, md=128: orig(-rp, nb, md)
        flipped = t5_float64(m.config, m.tensors, ids)
    finally:
        R.t5_bucket = orig
    assert np.abs(got - flipped).max() > 1e-2


def test_encoder_checks():
    m = synth.SyntheticT5("t5-tiny", 0, seed=3)
    with pytest.raises(RuntimeError, match="token id out of range"):
        R.t5_encode(m.config, m.tensors, np.array([0, m.config.vocab], np.int32))
    with pytest.raises(RuntimeError, match="te.0.wi.weight"):
        R.t5_encode(m.config, [t for t in m.tensors if t[0] != "te.0.wi.weight"], np.array([1, 2], np.int32))
