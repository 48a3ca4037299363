"""The T5 encoder (mgx_t5_*) on the GPU against the oracle's ref_t5_encode (t5.h:85-140), bit for
bit: every weight type, prompt lengths 1 to 256, the real T5-base shape, files written as
GGUF, buffer reuse across calls of different lengths, and the argument checks."""
import numpy as np
import pytest

from mgx import gguf as G
from mgx import synth
from oracle import cpu_ref as R

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def M():
    import mgx
    mgx.load()
    return mgx


def check(M, m, t5, seq, seed):
    ids = synth.synth_ids(seed, seq, m.config.vocab)
    got = t5.encode(ids)
    want = R.t5_encode(m.config, m.tensors, ids)
    assert np.array_equal(got, want), f"seq {seq}: max {np.abs(got - want).max()} at {np.argwhere(got != want)[:3]}"


@pytest.mark.parametrize("wtype", [0, 1, 8, 2])
def test_t5_tiny_matches_oracle(M, wtype):
    print(f"t5-tiny wtype={wtype}", flush=True)
    m = synth.SyntheticT5("t5-tiny", wtype, seed=5)
    t5 = M.T5(m.config, m.tensors)
    for seq in (1, 2, 7, 40, 64, 65, 130):
        check(M, m, t5, seq, seq)
    t5.close()


def test_t5_max_length(M):
    print("t5-tiny F16, 256 tokens", flush=True)
    m = synth.SyntheticT5("t5-tiny", 1, seed=6)
    t5 = M.T5(m.config, m.tensors)
    check(M, m, t5, 256, 3)
    check(M, m, t5, 5, 4)      # a short prompt after the longest: no stale rows or biases
    t5.close()


@pytest.mark.parametrize("wtype,seq", [(1, 24), (8, 13), (0, 70)])
def test_t5_mini_real_widths(M, wtype, seq):
    """One layer at T5-base's widths (768, 12 heads, 3072)."""
    print(f"t5-mini wtype={wtype} seq={seq}", flush=True)
    m = synth.SyntheticT5("t5-mini", wtype, seed=7)
    t5 = M.T5(m.config, m.tensors)
    check(M, m, t5, seq, 9)
    t5.close()


def test_t5_base_shape(M):
    """The full T5-base encoder shape (12 layers, 32128-entry vocab), F16 as converted."""
    print("t5-base F16, 24 tokens", flush=True)
    m = synth.SyntheticT5("t5-base", 1, seed=8)
    t5 = M.T5(m.config, m.tensors)
    check(M, m, t5, 24, 10)
    t5.close()


def test_t5_from_gguf(M, tmp_path):
    print("t5-tiny from GGUF", flush=True)
    m = synth.SyntheticT5("t5-tiny", 1, seed=11)
    p = tmp_path / "t5.gguf"
    G.write_t5(str(p), m)
    g = M.Gguf(p)
    t5 = M.T5.from_gguf(g)
    g.close()
    check(M, m, t5, 12, 12)
    t5.close()


def test_t5_checks(M):
    m = synth.SyntheticT5("t5-tiny", 1, seed=5)
    t5 = M.T5(m.config, m.tensors)
    with pytest.raises(M.MgxError, match="1 to 256 tokens"):
        t5.encode(np.zeros(0, np.int32))
    with pytest.raises(M.MgxError, match="1 to 256 tokens"):
        t5.encode(np.zeros(257, np.int32))
    with pytest.raises(M.MgxError, match="token id out of range"):
        t5.encode(np.array([1, m.config.vocab], np.int32))
    t5.close()
    with pytest.raises(M.MgxError, match="te.1.wo.weight"):
        M.T5(m.config, [t for t in m.tensors if t[0] != "te.1.wo.weight"])
    bad = synth.make_t5_config("t5-tiny", head_dim=32)
    with pytest.raises(M.MgxError, match="head_dim must be 64"):
        M.T5(bad, m.tensors)
