"""The oracle's LM forward and generation loop against an independent float64 numpy
restatement of lm_forward / lm_layer (src/mg/lm.h:152-259) on small models, plus the
invariants the reference relies on."""
import numpy as np
import pytest
from scipy.special import erf

from mgx import synth
from oracle import cpu_ref as R


def weights(m):
    W = {}
    for name, ttype, ne0, ne1, data in m.tensors:
        assert ttype == 0
        W[name] = data.view(np.float32).reshape(ne1, ne0).astype(np.float64)
    return W


def ln(x, w, b, eps=1e-5):
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * w + b


def attend(q, k, v, causal):
    # q [T, H, hd], k/v [U, H, hd]
    s = np.einsum("thd,uhd->htu", q, k) / np.sqrt(q.shape[-1])
    if causal:
        T, U = q.shape[0], k.shape[0]
        s = np.where(np.arange(U)[None, :] <= (np.arange(T) + U - T)[:, None], s, -np.inf)
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    return np.einsum("htu,uhd->thd", p, v)


def brute_forward(m, ids, t5, n_seq, cross):
    """float64 logits [n_seq][n_q][card] of the last of len(ids[0]) tokens fed at 0.."""
    c = m.config
    W = weights(m)
    d, H, hd, T = c.dim, c.heads, c.head_dim, ids.shape[1]
    i = np.arange(d // 2)
    pos = np.arange(T)[:, None] / np.power(c.max_period, i / c.pos_denominator)
    pe = np.concatenate([np.cos(pos), np.sin(pos)], 1).astype(np.float32).astype(np.float64)
    emb = sum(W[f"lm.emb.{q}.weight"][ids[q]] for q in range(c.n_q))
    x = np.repeat((pe + emb)[None], n_seq, 0)
    ctx = np.zeros((n_seq, t5.shape[0] if cross else 1, d))
    if cross:
        ctx[0] = t5.astype(np.float64) @ W["lm.cond_proj.weight"].T + W["lm.cond_proj.bias"][0]
    for l in range(c.layers):
        p = f"lm.{l}."
        nw = lambda k: (W[p + k + ".weight"][0], W[p + k + ".bias"][0])
        for n in range(n_seq):
            h = ln(x[n], *nw("norm1"))
            qkv = h @ W[p + "self.qkv.weight"].T
            q, k, v = (qkv[:, j * d:(j + 1) * d].reshape(T, H, hd) for j in range(3))
            x[n] = x[n] + attend(q, k, v, True).reshape(T, d) @ W[p + "self.out.weight"].T
            if cross:
                hc = ln(x[n], *nw("norm_cross"))
                cq = (hc @ W[p + "cross.q.weight"].T).reshape(T, H, hd)
                kv = ctx[n] @ W[p + "cross.kv.weight"].T
                ck, cv = kv[:, :d].reshape(-1, H, hd), kv[:, d:].reshape(-1, H, hd)
                x[n] = x[n] + attend(cq, ck, cv, False).reshape(T, d) @ W[p + "cross.out.weight"].T
            f = ln(x[n], *nw("norm2")) @ W[p + "ff.0.weight"].T
            f = 0.5 * f * (1 + erf(f / np.sqrt(2)))
            x[n] = x[n] + f @ W[p + "ff.2.weight"].T
    xl = ln(x[:, -1], W["lm.out_norm.weight"][0], W["lm.out_norm.bias"][0])
    return np.stack([np.stack([xl[n] @ W[f"lm.head.{q}.weight"].T for q in range(c.n_q)]) for n in range(n_seq)])


SMALL = dict(dim=64, layers=2, heads=4, ff_dim=256, card=32, n_ctx=3)


@pytest.mark.parametrize("shape,guided", [("tiny", True), ("tiny", False), (SMALL, True)])
def test_forward_matches_float64_brute_force(shape, guided):
    m = synth.SyntheticModel(shape, 0, seed=21, std=0.15)
    c = m.config
    t5 = synth.synth_memory(3, 5 if shape == "tiny" else 3)
    ids = synth.synth_codes(4, c.n_q, 9, c.card + 1)
    n_seq = 2 if guided else 1
    want = brute_forward(m, ids, t5, n_seq, guided)
    dec = R.RefDecoder(R.RefModel(c, m.tensors), 16, n_seq, t5 if guided else None, guided)
    got = dec.forward(ids)
    scale = np.abs(want).max()
    assert np.abs(got - want).max() <= 2e-5 * scale, np.abs(got - want).max() / scale
    # the first decode step after the prefill too
    ids2 = np.concatenate([ids, synth.synth_codes(5, c.n_q, 1, c.card + 1)], 1)
    want2 = brute_forward(m, ids2, t5, n_seq, guided)
    got2 = dec.forward(ids2[:, -1:])
    assert np.abs(got2 - want2).max() <= 2e-5 * np.abs(want2).max()


@pytest.fixture(scope="module")
def q8():
    m = synth.SyntheticModel("tiny", 8, seed=3)
    return m, R.RefModel(m.config, m.tensors)


def test_prefill_equals_incremental_and_hoisting(q8):
    m, rm = q8
    c = m.config
    t5 = synth.synth_memory(1, 5)
    ids = synth.synth_codes(2, c.n_q, 12, c.card)
    a = R.RefDecoder(rm, 40, 2, t5, True).forward(ids)
    d = R.RefDecoder(rm, 40, 2, t5, True, recompute_cross_kv=True)
    for t in range(12):
        b = d.forward(ids[:, t:t + 1])
    assert np.array_equal(a, b)
    # the null stream with zeroed memory equals a single unguided stream (lm.h:176-180)
    u = R.RefDecoder(rm, 40, 1, None, False).forward(ids)
    assert np.array_equal(a[1], u[0])


def test_decoder_errors_and_bookkeeping(q8):
    m, rm = q8
    c = m.config
    d = R.RefDecoder(rm, 6, 2, synth.synth_memory(1, 5), True)
    ids = synth.synth_codes(2, c.n_q, 5, c.card)
    d.forward(ids)
    assert d.used() == 5
    assert d.cache_bytes() == c.layers * 2 * 64 * 6 * c.heads * 2 * 4
    with pytest.raises(RuntimeError, match="prefill"):
        d.forward(ids[:, :2])
    d.forward(ids[:, :1])
    with pytest.raises(RuntimeError, match="overflow"):
        d.forward(ids[:, :1])


def test_generate_checks_and_first_logits(q8):
    m, rm = q8
    c = m.config
    t5 = synth.synth_memory(1, 5)
    prompt = synth.synth_codes(2, c.n_q, 6, c.card)
    with pytest.raises(RuntimeError, match="shorter"):
        rm.generate(t5, prompt, 6, 6)
    codes, first, rep, steps = rm.generate(t5, prompt, 6, 20, step_logits=True)
    assert np.array_equal(first, steps[0])
    assert (codes[:, :6] == prompt).all() and codes.min() >= 0 and codes.max() < c.card
    assert rep.prefill_tokens == 7 and rep.decode_steps == 20 + 4 - 7 - 1 and rep.forwards == 17
    # guidance on/off rule (pipeline.h:41-43, tests/conditioner_test.cpp:52-65)
    L = R.lib()
    assert [L.ref_use_guidance(3.0, 1), L.ref_use_guidance(3.0, 0), L.ref_use_guidance(0.0, 0),
            L.ref_use_guidance(0.0, 1)] == [0, 1, 0, 0]
    # an empty description generates unguided: same codes as cfg_coef 0
    a = rm.generate(t5, prompt, 6, 20, description_empty=True, seed=4)[0]
    b = rm.generate(t5, prompt, 6, 20, cfg_coef=0.0, seed=4)[0]
    assert np.array_equal(a, b)


def adapters_for(m, rank, strength, dora, seed=9):
    c = m.config
    rs = np.random.default_rng(seed)
    out = []
    for l in range(c.layers):
        for proj, (i, o) in {"self.qkv": (c.dim, 3 * c.dim), "ff.0": (c.dim, c.ff_dim), "ff.2": (c.ff_dim, c.dim)}.items():
            a = dict(target=f"lm.{l}.{proj}.weight", rank=rank, alpha=float(rank), strength=strength,
                     A=rs.normal(0, 0.01, (rank, i)).astype(np.float32),
                     B=rs.normal(0, 0.01, (o, rank)).astype(np.float32))
            if dora:
                a["magnitude"] = rs.uniform(0.9, 1.1, o).astype(np.float32)
            out.append(a)
    return out


@pytest.mark.parametrize("dora", [False, True])
def test_zero_strength_adapter_is_identity(q8, dora):
    """lora.h:58 / mg_train_parity_probe.cpp:97-102: strength 0 leaves the base model."""
    m, rm = q8
    c = m.config
    t5, ids = synth.synth_memory(1, 5), synth.synth_codes(2, c.n_q, 4, c.card)
    base = R.RefDecoder(rm, 8, 2, t5, True).forward(ids)
    ra = R.RefModel(c, m.tensors, adapters_for(m, 4, 0.0, dora))
    assert np.array_equal(R.RefDecoder(ra, 8, 2, t5, True).forward(ids), base)
    rb = R.RefModel(c, m.tensors, adapters_for(m, 4, 1.0, dora))
    assert not np.array_equal(R.RefDecoder(rb, 8, 2, t5, True).forward(ids), base)


def test_dora_rows_against_float64():
    """DoRA rows (lora.h:58-78): y = m / ||W + sBA||_row * (Wx + s B(Ax)) on an F32 base."""
    m = synth.SyntheticModel(SMALL, 0, seed=4, std=0.15)
    c = m.config
    ads = adapters_for(m, 4, 1.0, True, seed=5)
    rm = R.RefModel(c, m.tensors, ads)
    ids = synth.synth_codes(6, c.n_q, 3, c.card)
    got = R.RefDecoder(rm, 8, 1, None, False).forward(ids)
    # fold the adapters into dense weights and run the float64 brute force
    W = {t[0]: t for t in m.tensors}
    merged = synth.SyntheticModel(SMALL, 0, seed=4, std=0.15)
    for a in ads:
        name, ttype, ne0, ne1, data = W[a["target"]]
        w = data.view(np.float32).reshape(ne1, ne0).astype(np.float64)
        s = a["alpha"] / a["rank"]
        wd = w + s * (a["B"].astype(np.float64) @ a["A"].astype(np.float64))
        wd = wd * (a["magnitude"][:, None] / np.sqrt((wd ** 2).sum(1) + ne0 * 1e-12)[:, None])
        merged.replace(a["target"], 0, wd.astype(np.float32))
    want = brute_forward(merged, ids, None, 1, False)
    assert np.abs(got - want).max() <= 5e-5 * np.abs(want).max()


def test_timing_mode_runs_the_decode_steps_without_the_prefill():
    """The oracle's timing mode (the CPU baseline's sample of late decode steps) marks the
    prompt's positions as held by the cache instead of computing them: the decode steps then
    run at the same key counts, the prefill takes no time, and the mode switches back off."""
    m = synth.SyntheticModel("tiny", 8, seed=3)
    rm = R.RefModel(m.config, m.tensors)
    t5 = synth.synth_memory(1, 5)
    P, T = 40, 60
    prompt = synth.synth_codes(2, m.config.n_q, P, m.config.card)
    R.lib().ref_set_timing_history(1)
    try:
        codes, _, rep, _ = rm.generate(t5, prompt, P, T, seed=1, max_forwards=6)
    finally:
        R.lib().ref_set_timing_history(0)
    assert rep.forwards == 6 and rep.prefill_seconds < 1e-3
    assert np.array_equal(codes[:, :P], prompt)          # the prompt stays in the sequence
    # off again: the same call computes the prefill and matches a run that never used the mode
    c1, f1, rep1, _ = rm.generate(t5, prompt, P, T, seed=1)
    c2, f2, _, _ = R.RefModel(m.config, m.tensors).generate(t5, prompt, P, T, seed=1)
    assert rep1.forwards > 6 and np.array_equal(c1, c2) and np.array_equal(f1, f2)
