"""The oracle's sampling, RNG and delay-pattern restatements held to the reference:

* the golden vectors of the reference's own tests (tests/sampling_test.cpp:81-281 and
  tests/pattern_test.cpp:90-225, copied as data into tests/golden/*.json);
* the reference's own code for these functions (src/mg/sampling.h, src/rng.h,
  src/mg/pattern.h), compiled from its sources into oracle/_ref/ -- bit for bit on random
  rows, where that build exists;
* closed forms (std::mt19937's 10000th output is fixed by the C++ standard)."""
import ctypes as C
import json
import os
import subprocess

import numpy as np
import pytest

from oracle import cpu_ref as R

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
SAMPLING = json.load(open(os.path.join(GOLDEN, "sampling_cases.json")))["cases"]
PATTERN = json.load(open(os.path.join(GOLDEN, "pattern_cases.json")))["cases"]
L = R.lib()


def f32(a):
    return np.ascontiguousarray(a, np.float32)


@pytest.mark.parametrize("tag", sorted(SAMPLING))
def test_sampling_golden(tag):
    c = SAMPLING[tag]
    logits = f32(c["logits"])
    probs = np.zeros(c["n"], np.float32)
    L.ref_softmax_into(R.ptr(logits), c["n"], c["temperature"], R.ptr(probs))
    np.testing.assert_allclose(probs, c["softmax"], atol=1e-6, rtol=0)
    L.ref_top_k_filter(R.ptr(probs), c["n"], c["k"])
    np.testing.assert_allclose(probs, c["filtered"], atol=1e-6, rtol=0)
    assert int((probs > 0).sum()) == c["survivors"]
    assert abs(float(probs.astype(np.float64).sum()) - 1.0) <= 1e-5
    assert L.ref_argmax(R.ptr(logits), c["n"]) == c["argmax"]


def test_tie_at_cutoff_keeps_more_than_k():
    c = SAMPLING["TIED"]
    assert c["survivors"] > c["k"]


def test_sampling_draws_track_distribution():
    """sampling_test.cpp:208-247: draws stay in the surviving set and follow it."""
    c = SAMPLING["PLAIN"]
    logits = f32(c["logits"])
    rng = R.RefRng(7)
    scratch = np.zeros(c["n"], np.float32)
    counts = np.zeros(c["n"])
    draws = 50000
    for _ in range(draws):
        t = L.ref_sample_top_k(R.ptr(logits), c["n"], c["k"], c["temperature"], rng.buf, R.ptr(scratch))
        assert 0 <= t < c["n"] and c["filtered"][t] > 0
        counts[t] += 1
    assert np.abs(counts / draws - np.array(c["filtered"])).max() < 0.01


def test_temperature_zero_is_greedy_and_huge_logits_are_finite():
    c = SAMPLING["PLAIN"]
    logits = f32(c["logits"])
    rng = R.RefRng(1)
    scratch = np.zeros(c["n"], np.float32)
    assert L.ref_sample_top_k(R.ptr(logits), c["n"], c["k"], 0.0, rng.buf, R.ptr(scratch)) == c["argmax"]
    big = f32([1000.0, 1001.0, 999.0, -1000.0])
    p = np.zeros(4, np.float32)
    L.ref_softmax_into(R.ptr(big), 4, 1.0, R.ptr(p))
    assert np.isfinite(p).all() and abs(float(p.sum()) - 1.0) < 1e-5 and L.ref_argmax(R.ptr(big), 4) == 1


def test_mt19937_known_answer_and_uniform():
    """The C++ standard fixes mt19937's 10000th output for the default seed 5489."""
    r = R.RefRng(5489)
    for _ in range(9999):
        r.next()
    assert r.next() == 4123659995
    r = R.RefRng(3)
    u = [r.uniform() for _ in range(1000)]
    assert all(0.0 < x <= 1.0 for x in u)


@pytest.mark.parametrize("tag", sorted(PATTERN))
def test_pattern_golden(tag):
    c = PATTERN[tag]
    S = L.ref_pattern_steps(c["n_q"], c["timesteps"])
    assert S == c["steps"]
    codes = np.array(c["codes"], np.int32)
    seq = np.zeros(c["n_q"] * S, np.int32)
    L.ref_build_pattern(c["n_q"], c["timesteps"], R.ptr(codes), c["special"], R.ptr(seq))
    assert seq.tolist() == c["sequence"]
    back = np.zeros(c["n_q"] * c["timesteps"], np.int32)
    L.ref_revert_pattern(c["n_q"], c["timesteps"], R.ptr(np.array(c["sequence"], np.int32)), c["special"], R.ptr(back))
    assert back.tolist() == c["reverted"]
    mask = np.zeros(c["n_q"] * S, np.uint8)
    L.ref_pattern_mask(c["n_q"], c["timesteps"], R.ptr(mask))
    assert mask.tolist() == c["mask"]
    # first_step_with_timestep(t) = t + 1 for delays 0..n_q-1 (the loop's start offset)
    assert [t + 1 for t in range(c["timesteps"])] == c["first_step"]


def test_pattern_generation_invariants():
    """pattern_test.cpp:157-211 at the real shape: 1500 timesteps, a 6 s prompt."""
    assert L.ref_pattern_steps(4, 1500) == 1504
    S = 1504
    mask = np.zeros(4 * S, np.uint8)
    L.ref_pattern_mask(4, 1500, R.ptr(mask))
    mask = mask.reshape(4, S)
    assert (mask.sum(axis=1) == 1500).all()            # every codebook covers every timestep once
    assert S - (300 + 1) == 1203                        # 1203 forwards after a 300-timestep prompt
    codes = np.arange(4 * 1500, dtype=np.int32)
    seq = np.zeros(4 * S, np.int32)
    L.ref_build_pattern(4, 1500, R.ptr(codes), -7, R.ptr(seq))
    back = np.zeros(4 * 1500, np.int32)
    L.ref_revert_pattern(4, 1500, R.ptr(seq), -7, R.ptr(back))
    assert np.array_equal(back, codes)


# --- against the reference's own code, compiled from its sources -----------------------------
REFX = R.ref_host()
needs_ref = pytest.mark.skipif(REFX is None, reason="oracle/_ref not built (needs the reference tree)")


@needs_ref
def test_reference_own_unit_tests_pass():
    here = os.path.join(os.path.dirname(R.__file__), "_ref")
    for exe in ("sampling_test", "pattern_test"):
        out = subprocess.run([os.path.join(here, exe)], capture_output=True, text=True, timeout=120)
        assert out.returncode == 0, out.stderr


@needs_ref
@pytest.mark.parametrize("seed", range(6))
def test_softmax_topk_bit_exact_vs_reference(seed):
    rs = np.random.default_rng(seed)
    n = 2048
    logits = f32(rs.normal(0, 1 + seed, n))
    if seed % 2:
        logits[rs.integers(0, n, 50)] = logits[5]       # ties
    for temp in (1.0, 0.7, 2.5):
        a = np.zeros(n, np.float32)
        b = np.zeros(n, np.float32)
        L.ref_softmax_into(R.ptr(logits), n, temp, R.ptr(a))
        REFX.refx_softmax_into(R.ptr(logits), n, temp, R.ptr(b))
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        for k in (1, 50, 250, 2047, 0, 4096):
            x, y = a.copy(), b.copy()
            L.ref_top_k_filter(R.ptr(x), n, k)
            REFX.refx_top_k_filter(R.ptr(y), n, k)
            assert np.array_equal(x.view(np.uint32), y.view(np.uint32)), (temp, k)


@needs_ref
@pytest.mark.parametrize("k,temp", [(250, 1.0), (1, 1.0), (0, 1.0), (50, 0.5), (250, 0.0)])
def test_sample_stream_bit_exact_vs_reference(k, temp):
    rs = np.random.default_rng(11)
    rows, n = 300, 2048
    logits = f32(rs.normal(0, 2.0, (rows, n)))
    want = np.zeros(rows, np.int32)
    REFX.refx_sample_rows(R.ptr(logits), rows, n, k, temp, 1234, R.ptr(want))
    rng = R.RefRng(1234)
    scratch = np.zeros(n, np.float32)
    got = [L.ref_sample_top_k(R.ptr(logits[r]), n, k, temp, rng.buf, R.ptr(scratch)) for r in range(rows)]
    assert got == want.tolist()


@needs_ref
def test_rng_bit_exact_vs_reference():
    for seed in (0, 1, 1234, 2 ** 40 + 5):
        want = np.zeros(2000, np.uint32)
        REFX.refx_rng_raw(seed, 2000, R.ptr(want))
        r = R.RefRng(seed)
        assert [r.next() for _ in range(2000)] == want.tolist()
        wu = np.zeros(2000, np.float32)
        REFX.refx_rng_uniforms(seed, 2000, R.ptr(wu))
        r = R.RefRng(seed)
        assert np.array_equal(np.array([r.uniform() for _ in range(2000)], np.float32), wu)


@needs_ref
@pytest.mark.parametrize("n_q,T", [(4, 1), (4, 3), (4, 50), (1, 7), (3, 2)])
def test_pattern_bit_exact_vs_reference(n_q, T):
    S = L.ref_pattern_steps(n_q, T)
    assert S == REFX.refx_pattern_steps(n_q, T)
    codes = np.random.default_rng(T).integers(-1, 2048, n_q * T).astype(np.int32)
    a = np.zeros(n_q * S, np.int32)
    b = np.zeros(n_q * S, np.int32)
    L.ref_build_pattern(n_q, T, R.ptr(codes), 2048, R.ptr(a))
    REFX.refx_build_pattern(n_q, T, R.ptr(codes), 2048, R.ptr(b))
    assert np.array_equal(a, b)
    ma = np.zeros(n_q * S, np.uint8)
    mb = np.zeros(n_q * S, np.uint8)
    L.ref_pattern_mask(n_q, T, R.ptr(ma))
    REFX.refx_pattern_mask(n_q, T, R.ptr(mb))
    assert np.array_equal(ma, mb)
    ra = np.zeros(n_q * T, np.int32)
    rb = np.zeros(n_q * T, np.int32)
    L.ref_revert_pattern(n_q, T, R.ptr(a), 2048, R.ptr(ra))
    REFX.refx_revert_pattern(n_q, T, R.ptr(a), 2048, R.ptr(rb))
    assert np.array_equal(ra, rb)
    assert REFX.refx_first_step_with_timestep(n_q, T, T) == -1          # out of range is rejected
