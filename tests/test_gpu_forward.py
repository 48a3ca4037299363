"""HIP decode step vs the oracle, bit for bit, through the C ABI (mgx_forward)."""
import numpy as np
import pytest

from tests import helpers as H

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def mgx():
    import mgx as M
    M.load()
    return M


@pytest.mark.parametrize("wtype", [8, 2, 1, 0])
def test_tiny_forward_matches_oracle(mgx, wtype):
    from oracle import cpu_ref as R
    m = H.model("tiny", wtype, 3)
    c = m.config
    t5 = H.memory(1, 5)
    ids = H.codes(2, 4, 12, c.card)
    gm = mgx.Model(c, m.tensors)
    gs = mgx.Stream(gm, 40, 2, t5, True)
    rd = R.RefDecoder(H.ref_model("tiny", wtype, 3), 40, 2, t5, True)
    print(f"tiny forward wtype={wtype}: prefill 8 then 4 steps", flush=True)
    got = gs.forward(ids[:, :8])
    want = rd.forward(ids[:, :8])
    assert np.array_equal(got, want), f"prefill logits differ: max {np.abs(got - want).max()}"
    for t in range(8, 12):
        got = gs.forward(ids[:, t:t + 1])
        want = rd.forward(ids[:, t:t + 1])
        assert np.array_equal(got, want), f"step {t}: max {np.abs(got - want).max()}"
    assert gs.used() == 12 and gs.forwards() == 5


@pytest.mark.parametrize("shape,wtype", [("mini1024", 8), ("mini1024", 2), ("mini1024", 1), ("mini1024", 0),
                                         ("mini1536", 8), ("mini2048", 2), ("mini2048", 8)])
@pytest.mark.parametrize("n_seq", [1, 2, 3, 16])
def test_width_forward_matches_oracle(mgx, shape, wtype, n_seq):
    """The specialised GEMV shapes (dims 1024 / 1536 / 2048, ff 4x) and the column groups."""
    from oracle import cpu_ref as R
    m = H.model(shape, wtype, 4)
    c = m.config
    from mgx import synth
    t5 = H.memory(5, synth.SHAPES[shape]["n_ctx"])
    ids = H.codes(6, 4, 6, c.card)
    gm = mgx.Model(c, m.tensors)
    gs = mgx.Stream(gm, 16, n_seq, t5, True)
    rd = R.RefDecoder(H.ref_model(shape, wtype, 4), 16, n_seq, t5, True)
    print(f"{shape} wtype={wtype} n_seq={n_seq}: prefill 4 then 2 steps", flush=True)
    got = gs.forward(ids[:, :4])
    want = rd.forward(ids[:, :4])
    assert np.array_equal(got, want), f"prefill logits differ: max {np.abs(got - want).max()}"
    for t in range(4, 6):
        got = gs.forward(ids[:, t:t + 1])
        want = rd.forward(ids[:, t:t + 1])
        assert np.array_equal(got, want), f"step {t}: max {np.abs(got - want).max()}"


def test_many_streams_forward_matches_oracle(mgx):
    """Five streams: column groups 2 + 2 + 1 in every projection."""
    from oracle import cpu_ref as R
    m = H.model("tiny", 8, 3)
    c = m.config
    t5 = H.memory(1, 5)
    ids = H.codes(7, 4, 6, c.card)
    gs = mgx.Stream(mgx.Model(c, m.tensors), 16, 5, t5, True)
    rd = R.RefDecoder(H.ref_model("tiny", 8, 3), 16, 5, t5, True)
    print("tiny 5 streams", flush=True)
    assert np.array_equal(gs.forward(ids[:, :4]), rd.forward(ids[:, :4]))
    for t in range(4, 6):
        assert np.array_equal(gs.forward(ids[:, t:t + 1]), rd.forward(ids[:, t:t + 1]))


@pytest.mark.parametrize("wtype", [8, 2, 1, 0])
@pytest.mark.parametrize("n_seq", [1, 2, 4, 8])
def test_grouped_prefill_matches_oracle(mgx, wtype, n_seq):
    """A prefill runs its positions 512 / n_seq at a time (each column at its own position, causal
    by key count; the matrix-core GEMVs take the columns in 16-column groups, up to four per
    block against one load of the weights): prompts of 2, 17, 70, 257, 300, 512 and 600 tokens --
    one partial group, partial 16-column groups, several groups at every stream count, 256-key
    span boundaries inside a group, whole groups only (512 at every stream count) and one
    position past a whole guided group (257) -- then single steps, against the oracle's masked
    prefill (n_seq 3 and 16 keep one position at a time and are covered above)."""
    from oracle import cpu_ref as R
    m = H.model("tiny", wtype, 3)
    c = m.config
    t5 = H.memory(1, 5)
    gm = mgx.Model(c, m.tensors)
    for n_pre in (2, 17, 70, 257, 300, 512, 600):
        print(f"grouped prefill wtype={wtype} n_seq={n_seq} tokens={n_pre}", flush=True)
        ids = H.codes(n_pre, 4, n_pre + 2, c.card)
        gs = mgx.Stream(gm, n_pre + 4, n_seq, t5, True)
        rd = R.RefDecoder(H.ref_model("tiny", wtype, 3), n_pre + 4, n_seq, t5, True)
        got, want = gs.forward(ids[:, :n_pre]), rd.forward(ids[:, :n_pre])
        assert np.array_equal(got, want), f"prefill {n_pre}: max {np.abs(got - want).max()}"
        for t in range(n_pre, n_pre + 2):
            got, want = gs.forward(ids[:, t:t + 1]), rd.forward(ids[:, t:t + 1])
            assert np.array_equal(got, want), f"step {t}: max {np.abs(got - want).max()}"
        gs.close()
