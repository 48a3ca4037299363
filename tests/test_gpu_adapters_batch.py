"""Adapters (LoRA and DoRA rows, lora.h:50-83) and lockstep request batches on the GPU,
through the C ABI, against the oracle bit for bit."""
import numpy as np
import pytest

from mgx import synth
from tests import helpers as H

pytestmark = pytest.mark.gpu

ALL = ("self.qkv", "self.out", "cross.q", "cross.kv", "cross.out", "ff.0", "ff.2")
C5 = ("self.qkv", "ff.0", "ff.2")


@pytest.fixture(scope="module")
def M():
    import mgx
    mgx.load()
    return mgx


def ref_with(shape, wtype, seed, ads):
    from oracle import cpu_ref as R
    m = H.model(shape, wtype, seed)
    return R.RefModel(m.config, m.tensors, ads)


def forward_both(M, shape, wtype, seed, ads, n_seq=2, prefill=8, steps=4):
    from oracle import cpu_ref as R
    m = H.model(shape, wtype, seed)
    c = m.config
    t5 = H.memory(seed + 1, synth.SHAPES[shape]["n_ctx"])
    ids = H.codes(seed + 2, c.n_q, prefill + steps, c.card)
    gm = M.Model(c, m.tensors)
    if ads is not None:
        gm.set_adapters(ads)
    gs = M.Stream(gm, prefill + steps + 4, n_seq, t5, True)
    rd = R.RefDecoder(ref_with(shape, wtype, seed, ads), prefill + steps + 4, n_seq, t5, True)
    out = []
    for t0, t1 in [(0, prefill)] + [(t, t + 1) for t in range(prefill, prefill + steps)]:
        got, want = gs.forward(ids[:, t0:t1]), rd.forward(ids[:, t0:t1])
        out.append((t0, got, want))
    return out


@pytest.mark.parametrize("wtype", [8, 2, 1, 0])
@pytest.mark.parametrize("dora,strength", [(False, 1.0), (True, 1.0), (True, 0.5), (False, 0.7)])
def test_adapter_forward_matches_oracle(M, wtype, dora, strength):
    """Every target projection adapted: self and cross attention, ff, the cross K/V projected
    once at stream creation, the f32 copies of activation-form inputs."""
    print(f"adapter forward tiny wtype={wtype} dora={dora} strength={strength}", flush=True)
    c = H.model("tiny", wtype, 3).config
    ads = synth.synth_adapters(c, rank=8, targets=ALL, dora=dora, alpha=12.0, strength=strength, seed=7)
    for t, got, want in forward_both(M, "tiny", wtype, 3, ads):
        assert np.array_equal(got, want), f"position {t}: max {np.abs(got - want).max()}"


@pytest.mark.parametrize("shape,wtype", [("mini1536", 8), ("mini1024", 2), ("mini2048", 2)])
@pytest.mark.parametrize("rank", [5, 16, 64])
def test_adapter_ranks_at_real_widths(M, shape, wtype, rank):
    """The A x kernel at widths 1024-8192 (one to eight 1024-element groups per thread) and
    ranks that fill one, two and eight of B . (Ax)'s partials."""
    print(f"adapter ranks {shape} wtype={wtype} rank={rank}", flush=True)
    c = H.model(shape, wtype, 4).config
    ads = synth.synth_adapters(c, rank=rank, targets=ALL, dora=True, seed=rank)
    for t, got, want in forward_both(M, shape, wtype, 4, ads, n_seq=3, prefill=4, steps=2):
        assert np.array_equal(got, want), f"position {t}: max {np.abs(got - want).max()}"


@pytest.mark.parametrize("shape,wtype,rank", [("mini1536", 8, 16), ("mini2048", 2, 64), ("mini1024", 1, 16),
                                              ("mini1024", 0, 5)])
@pytest.mark.parametrize("dora", [False, True])
def test_adapter_wide_prefill_matches_oracle(M, shape, wtype, rank, dora):
    """A 40-token prefill with every projection adapted runs its first 39 positions through the
    prefill view: 78 columns (39 positions x 2 streams). Quantized weights: five 16-column groups
    in one matrix-core launch -- the last one ragged, blocks of several groups against one load
    of the weights, the adapter's A x staged group by group. F16 / F32 weights: the vector GEMV's
    whole column sets on blockIdx.y of one launch (each set's A x, sources and destinations
    advanced by its first column), then the ragged tail set in its own launch. Then single
    steps."""
    print(f"adapter wide prefill {shape} wtype={wtype} rank={rank} dora={dora}", flush=True)
    c = H.model(shape, wtype, 5).config
    ads = synth.synth_adapters(c, rank=rank, targets=ALL, dora=dora, seed=rank + 1)
    for t, got, want in forward_both(M, shape, wtype, 5, ads, prefill=40, steps=2):
        assert np.array_equal(got, want), f"position {t}: max {np.abs(got - want).max()}"


@pytest.mark.parametrize("dora", [False, True])
def test_zero_strength_adapter_is_identity(M, dora):
    """lora.h:62 / mg_train_parity_probe.cpp:97-102: strength 0 gives the base model bit for bit."""
    c = H.model("tiny", 8, 3).config
    base = forward_both(M, "tiny", 8, 3, None)
    zero = forward_both(M, "tiny", 8, 3, synth.synth_adapters(c, rank=4, targets=ALL, dora=dora, strength=0.0))
    for (t, g0, _), (_, g1, _) in zip(base, zero):
        assert np.array_equal(g0, g1), f"position {t}"


def test_adapter_errors_and_detach(M):
    m = H.model("tiny", 8, 3)
    c = m.config
    gm = M.Model(c, m.tensors)
    good = synth.synth_adapters(c, rank=4, targets=("ff.0",), dora=True)

    def expect(ads, code, text):
        with pytest.raises(M.MgxError) as e:
            gm.set_adapters(ads)
        assert e.value.code == code and text in str(e.value), str(e.value)

    bad = dict(good[0], target="lm.0.ff.1.weight")
    expect([bad], -1, "unsupported MusicGen adapter target")
    expect([dict(good[0], target=f"lm.{c.layers}.ff.0.weight")], -1, "unsupported MusicGen adapter target")
    expect([dict(good[0], alpha=0.0)], -1, "invalid adapter rank, alpha or strength")
    expect([dict(good[0], strength=float("inf"))], -1, "invalid adapter rank, alpha or strength")
    nan_b = good[0]["B"].copy()
    nan_b[3, 1] = np.nan
    expect([dict(good[0], B=nan_b)], -1, "nonfinite adapter tensor")
    expect([good[0], good[0]], -1, "two adapters")
    big = synth.synth_adapters(c, rank=65, targets=("ff.0",), dora=False)
    expect(big, -1, "ranks above 64")
    # a stream pins the adapters; after it is gone they can change, and n = 0 detaches
    t5 = H.memory(1, 5)
    ids = H.codes(2, c.n_q, 3, c.card)
    base = M.Stream(gm, 8, 2, t5, True).forward(ids)
    gm.set_adapters(good)
    s = M.Stream(gm, 8, 2, t5, True)
    adapted = s.forward(ids)
    assert not np.array_equal(adapted, base)
    expect([], -4, "no stream or session")
    s.close()
    gm.set_adapters([])
    assert np.array_equal(M.Stream(gm, 8, 2, t5, True).forward(ids), base)


# ---------------------------------------------------------------------------------------
# lockstep batches: every request equals mg_generate on that request alone
# ---------------------------------------------------------------------------------------
def batch_vs_oracle(M, shape, wtype, seed, reqs, prompt_len, T, ads=None):
    m = H.model(shape, wtype, seed)
    c = m.config
    n_ctx = synth.SHAPES[shape]["n_ctx"]
    gm = M.Model(c, m.tensors)
    if ads is not None:
        gm.set_adapters(ads)
    rm = ref_with(shape, wtype, seed, ads) if ads is not None else H.ref_model(shape, wtype, seed)
    requests = []
    for i, r in enumerate(reqs):
        requests.append(dict(t5=H.memory(100 + i, n_ctx), prompt=H.codes(200 + i, c.n_q, prompt_len, c.card),
                             params=M.GenerateParams(T, r.get("sampling", 1), r.get("temperature", 1.0),
                                                     r.get("top_k", 250), r.get("cfg", 3.0), r["seed"]),
                             description_empty=r.get("empty", False)))
    b = M.Batch(gm, requests, prompt_len, keep_step_logits=True)
    assert b.requests() == len(reqs)
    total = b.remaining()
    assert b.step(1) == 1 and b.remaining() == total - 1
    while b.remaining() > 0:
        b.step(7)
    for i, (q, r) in enumerate(zip(requests, reqs)):
        gc, gf, grep, gs = b.finish(i)
        p = q["params"]
        rc, rf, rrep, rs = rm.generate(q["t5"], q["prompt"], prompt_len, T, use_sampling=bool(p.use_sampling),
                                       temperature=p.temperature, top_k=p.top_k, cfg_coef=p.cfg_coef, seed=p.seed,
                                       description_empty=q["description_empty"], step_logits=True)
        step = H.first_diff(gs, rs)
        assert step is None, f"request {i}: mixed logits part at flat index {step} (step {step // gs[0].size})"
        assert np.array_equal(gf, rf), f"request {i}: first logits"
        assert np.array_equal(gc, rc), f"request {i}: codes"
        assert grep.forwards == rrep.forwards and grep.cache_bytes == rrep.cache_bytes
    b.close()


MIXED = [dict(seed=11), dict(seed=12, top_k=1, temperature=0.8, cfg=2.0), dict(seed=13, sampling=0),
         dict(seed=14, top_k=0, temperature=1.3, cfg=5.0)]


@pytest.mark.parametrize("wtype", [8, 1])
def test_batch_generate_matches_oracle(M, wtype):
    print(f"batch of 4 guided requests, tiny wtype={wtype}", flush=True)
    batch_vs_oracle(M, "tiny", wtype, 5, MIXED, 10, 40)


def test_unguided_batch_matches_oracle(M):
    """Unguided requests (cfg 0 or an empty description) run one stream each without
    cross-attention (pipeline.cpp:233-242)."""
    print("batch of 5 unguided requests, tiny Q8_0", flush=True)
    reqs = [dict(seed=21, cfg=0.0), dict(seed=22, empty=True), dict(seed=23, cfg=0.0, top_k=3),
            dict(seed=24, cfg=0.0, sampling=0), dict(seed=25, empty=True, temperature=0.5)]
    batch_vs_oracle(M, "tiny", 8, 6, reqs, 6, 30)


def test_batch_with_dora_adapters_matches_oracle(M):
    """The serving shape in small: 8 guided requests with rank-16 DoRA rows on qkv and the
    feed-forward, at the medium model's widths (one layer)."""
    print("batch of 8 guided requests with DoRA, mini1536 Q8_0", flush=True)
    c = H.model("mini1536", 8, 7).config
    ads = synth.synth_adapters(c, rank=16, targets=C5, dora=True, seed=3)
    reqs = [dict(seed=30 + i, top_k=250 if i % 2 == 0 else 20) for i in range(8)]
    batch_vs_oracle(M, "mini1536", 8, 7, reqs, 12, 40, ads)


def test_batch_rejects_mixed_or_oversized(M):
    m = H.model("tiny", 8, 5)
    c = m.config
    gm = M.Model(c, m.tensors)

    def req(i, cfg=3.0, T=20):
        return dict(t5=H.memory(i, 5), prompt=H.codes(i, c.n_q, 4, c.card), params=M.GenerateParams(T, 1, 1.0, 250, cfg, i))

    with pytest.raises(M.MgxError, match="all guided or all unguided"):
        M.Batch(gm, [req(1), req(2, cfg=0.0)], 4)
    with pytest.raises(M.MgxError, match="share max_gen_len"):
        M.Batch(gm, [req(1), req(2, T=21)], 4)
    with pytest.raises(M.MgxError, match="at most 16 streams"):
        M.Batch(gm, [req(i) for i in range(9)], 4)
    with pytest.raises(M.MgxError, match="1 to 16 requests"):
        M.Batch(gm, [req(i, cfg=0.0) for i in range(17)], 4)
    b = M.Batch(gm, [req(i, cfg=0.0) for i in range(16)], 4)
    assert b.requests() == 16
    with pytest.raises(M.MgxError, match="request index"):
        b.finish(16)
    b.close()
