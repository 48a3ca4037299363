"""Edge cases of the decode path on the GPU, through the C ABI, against the oracle bit for bit:
a stream reset and reused over stale cache rows (the reference fills its caches with N(0,1)
so a read past `used` shows, tests/kv_attention_test.cpp:96-103), the reference's two
Decoder::forward errors (KV overflow, kv_cache.h:73-77; a multi-token forward after history,
pipeline.cpp:81-83), prefill groups that end in a ragged 16-column group, and 16-column
decode steps attending many 64-key chunks."""
import numpy as np
import pytest

from mgx import synth
from tests import helpers as H

pytestmark = pytest.mark.gpu

ALL = ("self.qkv", "self.out", "cross.q", "cross.kv", "cross.out", "ff.0", "ff.2")


@pytest.fixture(scope="module")
def M():
    import mgx
    mgx.load()
    return mgx


@pytest.mark.parametrize("wtype", [8, 1])
def test_reset_over_stale_rows_matches_fresh_oracle(M, wtype):
    """A long sequence fills 300 rows of every cache (five 64-key chunks, two 256-key spans); after a reset a
    shorter, different sequence must give exactly what a fresh decoder gives: no row past the
    new position may leak into the attention, whatever it holds."""
    from oracle import cpu_ref as R
    m = H.model("tiny", wtype, 3)
    c = m.config
    t5 = H.memory(1, 5)
    gm = M.Model(c, m.tensors)
    gs = M.Stream(gm, 320, 2, t5, True)
    long_ids = H.codes(31, c.n_q, 300, c.card)
    print(f"stale rows wtype={wtype}: 290-token prefill + 10 steps, reset, 20 + 6", flush=True)
    gs.forward(long_ids[:, :290])
    for t in range(290, 300):
        gs.forward(long_ids[:, t:t + 1])
    assert gs.used() == 300
    forwards = gs.forwards()
    gs.reset()                       # KvCache::reset (kv_cache.h:70): used only
    assert gs.used() == 0 and gs.forwards() == forwards
    ids = H.codes(32, c.n_q, 26, c.card)
    rd = R.RefDecoder(H.ref_model("tiny", wtype, 3), 320, 2, t5, True)
    got, want = gs.forward(ids[:, :20]), rd.forward(ids[:, :20])
    assert np.array_equal(got, want), f"prefill after reset: max {np.abs(got - want).max()}"
    for t in range(20, 26):
        got, want = gs.forward(ids[:, t:t + 1]), rd.forward(ids[:, t:t + 1])
        assert np.array_equal(got, want), f"step {t} after reset: max {np.abs(got - want).max()}"
    # one position at a time from an empty cache, also over the stale rows
    gs.reset()
    rd2 = R.RefDecoder(H.ref_model("tiny", wtype, 3), 320, 2, t5, True)
    for t in range(4):
        got, want = gs.forward(ids[:, t:t + 1]), rd2.forward(ids[:, t:t + 1])
        assert np.array_equal(got, want), f"single step {t} after reset"


def test_forward_errors_are_the_references(M):
    """KV overflow (kv_cache.h:73-77) and a multi-token forward after history (pipeline.cpp:
    81-83) fail with their status, before any device work: the stream stays usable and still
    matches the oracle afterwards."""
    from oracle import cpu_ref as R
    m = H.model("tiny", 8, 3)
    c = m.config
    t5 = H.memory(1, 5)
    gs = M.Stream(M.Model(c, m.tensors), 8, 2, t5, True)
    rd = R.RefDecoder(H.ref_model("tiny", 8, 3), 8, 2, t5, True)
    ids = H.codes(41, c.n_q, 9, c.card)
    assert np.array_equal(gs.forward(ids[:, :5]), rd.forward(ids[:, :5]))
    with pytest.raises(M.MgxError) as e:
        gs.forward(ids[:, 5:7])
    assert e.value.code == -4, str(e.value)
    assert gs.used() == 5
    for t in range(5, 8):
        assert np.array_equal(gs.forward(ids[:, t:t + 1]), rd.forward(ids[:, t:t + 1])), f"step {t}"
    with pytest.raises(M.MgxError) as e:
        gs.forward(ids[:, 8:9])
    assert e.value.code == -3, str(e.value)
    assert gs.used() == 8
    # a prefill longer than the capacity overflows too
    gs2 = M.Stream(M.Model(c, m.tensors), 4, 2, t5, True)
    with pytest.raises(M.MgxError) as e:
        gs2.forward(ids[:, :5])
    assert e.value.code == -3, str(e.value)
    assert gs2.used() == 0


def forward_pair(M, shape, wtype, seed, ads, n_seq, prefill, steps):
    from oracle import cpu_ref as R
    m = H.model(shape, wtype, seed)
    c = m.config
    t5 = H.memory(seed + 1, synth.SHAPES[shape]["n_ctx"])
    ids = H.codes(seed + 2, c.n_q, prefill + steps, c.card)
    gm = M.Model(c, m.tensors)
    if ads is not None:
        gm.set_adapters(ads)
    rm = R.RefModel(c, m.tensors, ads)
    gs = M.Stream(gm, prefill + steps + 4, n_seq, t5, True)
    rd = R.RefDecoder(rm, prefill + steps + 4, n_seq, t5, True)
    for t0, t1 in [(0, prefill)] + [(t, t + 1) for t in range(prefill, prefill + steps)]:
        got, want = gs.forward(ids[:, t0:t1]), rd.forward(ids[:, t0:t1])
        assert np.array_equal(got, want), f"positions {t0}..{t1 - 1}: max {np.abs(got - want).max()}"


@pytest.mark.parametrize("n_seq,prefill", [(2, 20), (2, 52), (1, 30)])
@pytest.mark.parametrize("dora", [False, True])
def test_ragged_wide_group_with_adapters(M, n_seq, prefill, dora):
    """Prefill groups whose last 16-column group is only partly live: 19 positions x 2 streams
    = 38 columns, 32 + 19 positions (64 + 38 columns; the c5 prompts end the same way), and 29
    columns of one stream -- every projection adapted, at the medium width (matrix-core GEMVs)."""
    print(f"ragged wide group n_seq={n_seq} prefill={prefill} dora={dora}", flush=True)
    c = H.model("mini1536", 8, 5).config
    ads = synth.synth_adapters(c, rank=16, targets=ALL, dora=dora, seed=prefill)
    forward_pair(M, "mini1536", 8, 5, ads, n_seq, prefill, 2)


@pytest.mark.parametrize("dora", [False, True])
def test_sixteen_columns_over_several_chunks(M, dora):
    """The batched serving shape in small: 8 guided requests (16 columns per step) with a
    300-frame prompt and 600 frames in all, so decode steps attend up to 603 keys: ten
    64-key chunks at 16 columns, each request against its own oracle generation."""
    from oracle import cpu_ref as R
    print(f"8 guided requests x 600 frames, tiny Q8_0, dora={dora}", flush=True)
    m = H.model("tiny", 8, 9)
    c = m.config
    gm = M.Model(c, m.tensors)
    ads = synth.synth_adapters(c, rank=16, targets=("self.qkv", "ff.0", "ff.2"), dora=True, seed=4) if dora else None
    if ads is not None:
        gm.set_adapters(ads)
    rm = R.RefModel(c, m.tensors, ads)
    P, T = 300, 600
    reqs = []
    for i in range(8):
        reqs.append(dict(t5=H.memory(300 + i, 5), prompt=H.codes(400 + i, c.n_q, P, c.card),
                         params=M.GenerateParams(T, 1, 1.0, 250 if i % 2 == 0 else 20, 3.0, 50 + i),
                         description_empty=False))
    b = M.Batch(gm, reqs, P, keep_step_logits=True)
    while b.remaining() > 0:
        b.step(64)
    for i, q in enumerate(reqs):
        gc, gf, _, gst = b.finish(i)
        p = q["params"]
        rc, rf, _, rst = rm.generate(q["t5"], q["prompt"], P, T, use_sampling=True, temperature=1.0, top_k=p.top_k,
                                     cfg_coef=3.0, seed=p.seed, step_logits=True)
        step = H.first_diff(gst, rst)
        assert step is None, f"request {i}: mixed logits part at step {step // gst[0].size}"
        assert np.array_equal(gf, rf) and np.array_equal(gc, rc), f"request {i}"
    b.close()


@pytest.mark.parametrize("n_ctx", [1, 32, 33, 64, 65, 200])
def test_memory_lengths_across_the_cross_attention_kernels(M, n_ctx):
    """Conditioning of 1-32 tokens runs the 32-key cross-attention wave, 33-64 the 64-key wave,
    65-256 the 256-thread kernel (lm.h:181-199): each against the oracle, prefill and steps."""
    from oracle import cpu_ref as R
    print(f"memory of {n_ctx} tokens, tiny Q8_0", flush=True)
    m = H.model("tiny", 8, 11)
    c = m.config
    t5 = H.memory(12, n_ctx)
    ids = H.codes(13, c.n_q, 10, c.card)
    gs = M.Stream(M.Model(c, m.tensors), 16, 2, t5, True)
    rd = R.RefDecoder(H.ref_model("tiny", 8, 11), 16, 2, t5, True)
    for t0, t1 in [(0, 6)] + [(t, t + 1) for t in range(6, 10)]:
        got, want = gs.forward(ids[:, t0:t1]), rd.forward(ids[:, t0:t1])
        assert np.array_equal(got, want), f"positions {t0}..{t1 - 1}: max {np.abs(got - want).max()}"
