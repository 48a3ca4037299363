"""mg_generate on the GPU (mgx_generate / sessions) against the oracle's restatement.

Live cases run the oracle beside the GPU on small shapes and compare every step's mixed
logits bit for bit; fixture cases replay the four single-request workloads (small Q8_0 and F16,
medium Q8_0, large Q4_0) at full length against codes the oracle produced ahead of time
(tests/golden/make_fixtures.py)."""
import os
import zlib

import numpy as np
import pytest

from tests import helpers as H

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def M():
    import mgx
    mgx.load()
    return mgx


def run_both(M, shape, wtype, seed, prompt_len, T, sampling, top_k, temperature=1.0, cfg=3.0, description_empty=False):
    m = H.model(shape, wtype, seed)
    c = m.config
    n_ctx = M.SHAPES[shape]["n_ctx"]
    t5 = H.memory(seed, n_ctx)
    prompt = H.codes(seed, c.n_q, prompt_len, c.card)
    params = M.GenerateParams(T, 1 if sampling else 0, temperature, top_k, cfg, seed)
    g = M.Model(c, m.tensors).generate(t5, prompt, prompt_len, params, description_empty, step_logits=True)
    r = H.ref_model(shape, wtype, seed).generate(t5, prompt, prompt_len, T, use_sampling=sampling,
                                                  temperature=temperature, top_k=top_k, cfg_coef=cfg, seed=seed,
                                                  description_empty=description_empty, step_logits=True)
    return g, r


@pytest.mark.parametrize("wtype", [8, 2, 1])
@pytest.mark.parametrize("sampling,top_k", [(False, 250), (True, 250), (True, 1), (True, 0)])
def test_tiny_generate_matches_oracle(M, wtype, sampling, top_k):
    print(f"tiny generate wtype={wtype} sampling={sampling} top_k={top_k}", flush=True)
    (gc, gf, grep, gs), (rc, rf, rrep, rs) = run_both(M, "tiny", wtype, 5, 10, 40, sampling, top_k)
    step = H.first_diff(gs, rs)
    assert step is None, f"mixed logits part at flat index {step} (step {step // gs[0].size})"
    assert np.array_equal(gf, rf)
    assert np.array_equal(gc, rc)
    assert grep.forwards == rrep.forwards == 40 + 4 - 11
    assert grep.decode_steps == rrep.decode_steps and grep.prefill_tokens == rrep.prefill_tokens == 11
    assert grep.cache_bytes == rrep.cache_bytes


@pytest.mark.parametrize("wtype", [8, 1])
def test_tiny_long_generate_crosses_attention_chunks(M, wtype):
    """700 positions: three 256-key attention chunks, a graph per chunk count, prefill across a
    chunk boundary."""
    print(f"tiny long generate wtype={wtype}: prompt 300, 700 frames", flush=True)
    (gc, gf, _, gs), (rc, rf, _, rs) = run_both(M, "tiny", wtype, 11, 300, 700, True, 250)
    step = H.first_diff(gs, rs)
    assert step is None, f"mixed logits part at flat index {step} (step {step // gs[0].size})"
    assert np.array_equal(gf, rf) and np.array_equal(gc, rc)


def test_tiny_unguided_and_no_prompt(M):
    print("tiny generate: empty description (unguided), then no prompt", flush=True)
    (gc, gf, _, gs), (rc, rf, _, rs) = run_both(M, "tiny", 8, 6, 7, 30, True, 250, description_empty=True)
    assert np.array_equal(gs, rs) and np.array_equal(gc, rc)
    (gc, gf, _, gs), (rc, rf, _, rs) = run_both(M, "tiny", 8, 7, 0, 20, True, 250)
    assert np.array_equal(gs, rs) and np.array_equal(gc, rc)


def test_tiny_temperature_and_cfg_variants(M):
    print("tiny generate: temperature 0.7 / 0 and cfg 1.5", flush=True)
    for temp, cfg in ((0.7, 3.0), (0.0, 3.0), (1.3, 1.5)):
        (gc, _, _, gs), (rc, _, _, rs) = run_both(M, "tiny", 8, 8, 9, 30, True, 50, temperature=temp, cfg=cfg)
        assert np.array_equal(gs, rs) and np.array_equal(gc, rc), (temp, cfg)


def test_session_steps_equal_one_call(M):
    """Cutting the loop into sessions' steps changes nothing."""
    m = H.model("tiny", 8, 9)
    c = m.config
    t5, prompt = H.memory(9, 5), H.codes(9, c.n_q, 6, c.card)
    params = M.GenerateParams(25, 1, 1.0, 100, 3.0, 9)
    gm = M.Model(c, m.tensors)
    whole = gm.generate(t5, prompt, 6, params, step_logits=True)
    s = M.Session(gm, t5, prompt, 6, params, keep_step_logits=True)
    assert s.step(1) == 1
    while s.remaining():
        s.step(3)
    parts = s.finish()
    assert np.array_equal(whole[0], parts[0]) and np.array_equal(whole[3], parts[3])
    assert np.array_equal(whole[1], parts[1])


def _fixture(name):
    p = os.path.join(GOLDEN, name + ".npz")
    if not os.path.exists(p):
        pytest.skip(f"fixture {name} not generated")
    return np.load(p, allow_pickle=False)


FIXTURE_CASES = ["c1_small_q8", "c1_small_q8_greedy", "c2_small_f16_topk1", "c3_medium_q8", "c4_large_q4"]


@pytest.mark.slow
@pytest.mark.parametrize("name", FIXTURE_CASES)
def test_full_length_generation_matches_fixture(M, name):
    import sys
    sys.path.insert(0, GOLDEN)
    from make_fixtures import CASES, inputs, model_digest
    from oracle import cpu_ref as R
    f = _fixture(name)
    assert int(f["convention"]) == R.lib().ref_convention(), "fixture predates the current reduction order"
    case = CASES[name]
    print(f"full-length generation {name}", flush=True)
    m, t5, prompt = inputs(case)
    assert zlib.crc32(t5.tobytes()) == int(f["t5_crc"]) and zlib.crc32(prompt.tobytes()) == int(f["prompt_crc"])
    assert bytes(f["model_sha256"]).hex() == model_digest(m), "the synthetic generator changed; regenerate fixtures"
    T = case["prompt"] + case["gen"]
    params = M.GenerateParams(T, 1 if case["sampling"] else 0, 1.0, case["top_k"], 3.0, case["seed"])
    codes, first, rep, steps = M.Model(m.config, m.tensors).generate(t5, prompt, case["prompt"], params,
                                                                      step_logits=True)
    crc = np.array([zlib.crc32(steps[i].tobytes()) for i in range(steps.shape[0])], np.uint32)
    bad = np.nonzero(crc != f["step_crc"])[0]
    agree = float((codes == f["codes"]).mean())
    gen = codes[:, case["prompt"]:] == f["codes"][:, case["prompt"]:]
    print(f"  {name}: first differing step {bad[0] if bad.size else None}, code agreement {agree:.6f}, "
          f"generated-code agreement {gen.mean():.6f}, decode {rep.decode_steps / rep.decode_seconds:.1f} frames/s",
          flush=True)
    assert np.array_equal(first, f["first_logits"])
    assert gen.mean() >= 0.995
    assert bad.size == 0, f"mixed logits first differ at step {bad[0]}"


@pytest.mark.slow
def test_c5_batch_matches_fixture(M):
    """The batched serving workload at full size: 8 guided medium Q8_0 requests (16 columns, 48
    layers, rank-16 DoRA rows on qkv / ff.0 / ff.2), 500-frame prompts prefilled through the
    512-column view (256 positions, then a ragged group of 243), then 1502 decode steps attending up to 2003 keys (32
    64-key chunks at 16 columns): every request's mixed logits at every step (CRC), first
    logits and codes equal the oracle's generation of that request alone."""
    import sys
    sys.path.insert(0, GOLDEN)
    from make_fixtures import CASES, adapter_digest, batch_inputs, model_digest
    from oracle import cpu_ref as R
    name = "c5_medium_q8_batch8_dora"
    f = _fixture(name)
    assert int(f["convention"]) == R.lib().ref_convention(), "fixture predates the current reduction order"
    case = CASES[name]
    print(f"full-length batch {name}", flush=True)
    m, ads, reqs = batch_inputs(case)
    assert bytes(f["model_sha256"]).hex() == model_digest(m), "the synthetic generator changed; regenerate fixtures"
    assert bytes(f["adapter_sha256"]).hex() == adapter_digest(ads)
    T = case["prompt"] + case["gen"]
    requests = []
    for r, (t5, prompt, seed) in enumerate(reqs):
        assert zlib.crc32(t5.tobytes()) == int(f["t5_crc"][r]) and zlib.crc32(prompt.tobytes()) == int(f["prompt_crc"][r])
        requests.append(dict(t5=t5, prompt=prompt, params=M.GenerateParams(T, 1, 1.0, case["top_k"], 3.0, seed),
                             description_empty=False))
    gm = M.Model(m.config, m.tensors)
    gm.set_adapters(ads)
    b = M.Batch(gm, requests, case["prompt"], keep_step_logits=True)
    while b.remaining() > 0:
        b.step(256)
    for r in range(len(reqs)):
        codes, first, rep, steps = b.finish(r)
        crc = np.array([zlib.crc32(steps[i].tobytes()) for i in range(steps.shape[0])], np.uint32)
        bad = np.nonzero(crc != f["step_crc"][r])[0]
        print(f"  request {r}: first differing step {bad[0] if bad.size else None}", flush=True)
        assert np.array_equal(first, f["first_logits"][r]), f"request {r}: first logits"
        assert bad.size == 0, f"request {r}: mixed logits first differ at step {bad[0]}"
        assert np.array_equal(codes, f["codes"][r]), f"request {r}: codes"
    b.close()
