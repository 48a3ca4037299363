"""The request server (mgx_server_*) on the GPU: concurrent callers whose requests join and
leave one batched decode, each result equal to mgx_generate on that request alone (which the
generation tests pin to the oracle), plus one mixed case against the oracle directly."""
import threading

import numpy as np
import pytest

from mgx import synth
from tests import helpers as H

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def M():
    import mgx
    mgx.load()
    return mgx


def request(M, c, i, T, P, n_ctx, cfg=3.0, empty=False, sampling=1, top_k=250, temperature=1.0):
    return dict(t5=H.memory(100 + i, n_ctx), prompt=H.codes(200 + i, c.n_q, P, c.card), P=P, empty=empty,
                params=M.GenerateParams(T, sampling, temperature, top_k, cfg, 1000 + i))


def serve(M, gm, reqs, slots, guided=True, steps_per_round=0, late=()):
    """Every request from its own thread. The requests not in `late` are released together
    (a barrier); the `late` ones once request 0 has reported its third loop iteration, so they
    join a batch in flight. Returns the results, each request's progress calls and the
    server's counters."""
    T = max(r["params"].max_gen_len for r in reqs)
    ctx = max(r["t5"].shape[0] for r in reqs)
    srv = M.Server(gm, slots, T, max_ctx=ctx, guided=guided, keep_step_logits=True,
                   steps_per_round=steps_per_round)
    out, errors = [None] * len(reqs), []
    progress = [[] for _ in reqs]
    early = threading.Barrier(len(reqs) - len(late))
    mid = threading.Event()

    def note(i, d, t):
        progress[i].append((d, t))
        if i == 0 and d >= 3:
            mid.set()

    def work(i):
        r = reqs[i]
        try:
            if i in late:
                assert mid.wait(120)
            else:
                early.wait(60)
            out[i] = srv.generate(r["t5"], r["prompt"], r["P"], r["params"], description_empty=r["empty"],
                                  step_logits=True, progress=lambda d, t: note(i, d, t))
        except Exception as e:   # noqa: BLE001 -- reported below
            errors.append((i, e))

    threads = [threading.Thread(target=work, args=(i,)) for i in range(len(reqs))]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=300)
        assert not th.is_alive(), "a request did not finish"
    counters = srv.counters()
    srv.close()
    assert not errors, errors
    return out, progress, counters


def check_alone(M, gm, reqs, out, progress):
    for i, r in enumerate(reqs):
        codes, first, rep, steps = out[i]
        w_codes, w_first, w_rep, w_steps = gm.generate(r["t5"], r["prompt"], r["P"], r["params"],
                                                       description_empty=r["empty"], step_logits=True)
        assert np.array_equal(steps, w_steps), f"request {i}: step logits differ from row {H.first_diff(steps, w_steps)}"
        assert np.array_equal(first, w_first), f"request {i}: first logits"
        assert np.array_equal(codes, w_codes), f"request {i}: codes"
        total = r["params"].max_gen_len + gm.config.n_q - (r["P"] + 1)
        assert progress[i] == [(k, total) for k in range(1, total + 1)], f"request {i}: progress"
        assert (rep.prefill_tokens, rep.decode_steps, rep.forwards) == (w_rep.prefill_tokens, w_rep.decode_steps,
                                                                        w_rep.forwards)


def mixed(M, c):
    """Guided and unguided requests of different prompt, generation and conditioning lengths,
    greedy and sampled, different top-k, temperatures and guidance strengths."""
    return [request(M, c, 0, 60, 6, 5),
            request(M, c, 1, 22, 0, 3, cfg=0.0),
            request(M, c, 2, 40, 12, 9, top_k=7, temperature=0.7),
            request(M, c, 3, 18, 3, 4, empty=True),
            request(M, c, 4, 26, 9, 1, sampling=0),
            request(M, c, 5, 35, 1, 7, cfg=1.5, top_k=1),
            request(M, c, 6, 20, 5, 6, cfg=0.0, top_k=40)]


@pytest.mark.parametrize("wtype", [8, 2, 1])
@pytest.mark.parametrize("slots,steps_per_round", [(3, 4), (4, 0)])
def test_server_requests_equal_alone(M, wtype, slots, steps_per_round):
    """Seven requests through fewer slots: requests queue, join mid-flight and leave at their
    own ends (Q8_0 on the matrix cores, Q4_0 and F16 on the vector GEMV in column pairs)."""
    print(f"server tiny wtype={wtype} slots={slots} steps_per_round={steps_per_round}", flush=True)
    m = H.model("tiny", wtype, 11)
    gm = M.Model(m.config, m.tensors)
    reqs = mixed(M, m.config)
    out, progress, counters = serve(M, gm, reqs, slots, steps_per_round=steps_per_round, late=(5, 6))
    check_alone(M, gm, reqs, out, progress)
    assert counters["served"] == len(reqs) and counters["active"] == 0 and counters["queued"] == 0
    # several requests shared steps
    assert counters["slot_steps"] > counters["steps"]


def test_server_mixed_matches_oracle(M):
    """The same mix against the oracle's mg_generate directly."""
    print("server tiny Q8_0 vs oracle", flush=True)
    from oracle import cpu_ref as R
    m = H.model("tiny", 8, 12)
    gm = M.Model(m.config, m.tensors)
    reqs = mixed(M, m.config)[:5]
    out, _, _ = serve(M, gm, reqs, 2, steps_per_round=5, late=(4,))
    rm = R.RefModel(m.config, m.tensors)
    for i, r in enumerate(reqs):
        p = r["params"]
        codes, first, rep, steps = rm.generate(r["t5"], r["prompt"], r["P"], p.max_gen_len, use_sampling=bool(p.use_sampling),
                                               temperature=p.temperature, top_k=p.top_k, cfg_coef=p.cfg_coef, seed=p.seed,
                                               description_empty=r["empty"], step_logits=True)
        assert np.array_equal(out[i][3], steps), f"request {i}"
        assert np.array_equal(out[i][0], codes), f"request {i}"


def test_unguided_server_sixteen_slots(M):
    print("unguided server, 16 slots, tiny Q8_0", flush=True)
    m = H.model("tiny", 8, 13)
    c = m.config
    gm = M.Model(c, m.tensors)
    reqs = [request(M, c, 20 + i, 12 + 2 * i, i % 5, 4, cfg=0.0 if i % 2 else 3.0, empty=i % 2 == 0,
                    top_k=[250, 5, 1][i % 3]) for i in range(18)]
    out, progress, counters = serve(M, gm, reqs, 16, guided=False, late=(17,))
    check_alone(M, gm, reqs, out, progress)
    assert counters["served"] == 18


def test_server_with_dora_adapters_at_medium_width(M):
    """The serving shape in small: 8 slots of guided requests, rank-16 DoRA rows on qkv and the
    feed-forward, the medium model's widths (one layer), two requests arriving mid-flight."""
    print("server with DoRA, mini1536 Q8_0, 8 slots", flush=True)
    m = H.model("mini1536", 8, 14)
    c = m.config
    gm = M.Model(c, m.tensors)
    gm.set_adapters(synth.synth_adapters(c, rank=16, targets=("self.qkv", "ff.0", "ff.2"), dora=True, seed=4))
    reqs = [request(M, c, 40 + i, 16 + 3 * i, 2 + i, synth.SHAPES["mini1536"]["n_ctx"], top_k=250 if i % 2 else 20)
            for i in range(10)]
    out, progress, counters = serve(M, gm, reqs, 8, steps_per_round=6, late=(8, 9))
    check_alone(M, gm, reqs, out, progress)
    assert counters["slot_steps"] > counters["steps"]


def test_server_dora_long_prompts_prefill_in_wide_groups(M):
    """Admissions with DoRA rows and prompts past one prefill group (256 positions x 2 streams):
    each slot's prompt runs through the aimed view in a full group and a ragged one."""
    print("server with DoRA, long prompts, mini1536 Q8_0, 4 slots", flush=True)
    m = H.model("mini1536", 8, 15)
    c = m.config
    gm = M.Model(c, m.tensors)
    gm.set_adapters(synth.synth_adapters(c, rank=16, targets=("self.qkv", "ff.0", "ff.2"), dora=True, seed=5))
    n_ctx = synth.SHAPES["mini1536"]["n_ctx"]
    reqs = [request(M, c, 60, 278, 270, n_ctx), request(M, c, 61, 272, 265, n_ctx, top_k=20),
            request(M, c, 62, 20, 5, n_ctx)]
    out, progress, counters = serve(M, gm, reqs, 4)
    check_alone(M, gm, reqs, out, progress)


def test_server_checks_and_shutdown(M):
    m = H.model("tiny", 8, 15)
    c = m.config
    gm = M.Model(c, m.tensors)
    with pytest.raises(M.MgxError, match="at most 16 streams"):
        M.Server(gm, 9, 20)
    srv = M.Server(gm, 1, 20, max_ctx=5, guided=False)
    r = request(M, c, 1, 20, 4, 5)
    with pytest.raises(M.MgxError, match="needs slots of two streams"):
        srv.generate(r["t5"], r["prompt"], 4, r["params"])
    srv.close()
    srv = M.Server(gm, 1, 20, max_ctx=5)
    with pytest.raises(M.MgxError, match="above the server's limit"):
        q = request(M, c, 2, 21, 4, 5)
        srv.generate(q["t5"], q["prompt"], 4, q["params"])
    with pytest.raises(M.MgxError, match="conditioning longer"):
        q = request(M, c, 3, 20, 4, 6)
        srv.generate(q["t5"], q["prompt"], 4, q["params"])
    with pytest.raises(M.MgxError, match="keeps no per-step logits"):
        srv.generate(r["t5"], r["prompt"], 4, r["params"], step_logits=True)
    bad = r["prompt"].copy()
    bad[0, 0] = c.card
    with pytest.raises(M.MgxError, match="prompt code out of range"):
        srv.generate(r["t5"], bad, 4, r["params"])
    with pytest.raises(M.MgxError, match="adapter"):
        gm.set_adapters(synth.synth_adapters(c, rank=4, targets=("ff.0",), dora=False, seed=1))
    # shutting down with a request in flight and one queued: both callers get an error
    started = threading.Event()
    errors = []

    def work(T):
        q = request(M, c, 5, T, 2, 5)
        try:
            srv.generate(q["t5"], q["prompt"], 2, q["params"], progress=lambda d, t: started.set())
        except M.MgxError as e:
            errors.append(str(e))

    srv2 = M.Server(gm, 1, 4000, max_ctx=5, steps_per_round=2)
    srv, old = srv2, srv
    old.close()
    ths = [threading.Thread(target=work, args=(3990,)), threading.Thread(target=work, args=(3990,))]
    for th in ths:
        th.start()
    assert started.wait(120)
    srv.close()
    for th in ths:
        th.join(timeout=60)
        assert not th.is_alive()
    assert len(errors) == 2 and all("shut down" in e for e in errors), errors
