#!/usr/bin/env python3
"""Benchmark: MusicGen LM decode frames/s (and HBM GB/s) on one MI355X.

A step is one decode forward of the LM -- one delay-pattern sequence step, 4 codes, 20 ms of
audio -- including the on-device CFG mix and top-k sampling, exactly the loop body of the
reference's mg_generate (src/mg/pipeline.cpp:255-302). The workload is MusicGen-medium-shaped
(48 layers, dim 1536, 24 heads, FFN 6144, 4 x 2048 codebooks) with random N(0, 0.02) weights
quantized to Q8_0, CFG 3 over two streams, a 24 x 768 N(0,1) memory, a 500-frame random-code
prompt (prefilled, untimed) and a 1500-frame continuation sampled with top-k 250, temperature 1,
seed 1. W warmup decode steps run untimed, then exactly K decode steps are timed; a run of fewer
steps than the continuation holds is centred on the continuation's middle (the steps before it
run untimed), so the keys it attends average those of the whole 30 s continuation; if the
continuation runs out, a fresh session is prefilled outside the timed segments.

Prints one JSON line. `value` is decode frames/s over the timed steps (graph replays, nothing
else in the timed region). After them, untimed, the launches of a few decode steps at the timed
segment's middle stamp their spans on the GPU wall clock (earliest block start to latest wave
end, on the session's own stream): `roofline` is the dominant kernel's achieved HBM bandwidth
(algorithmic bytes per launch -- weights at their stored precision, 34/32 B per Q8_0 weight; for
attention the f32 K and V of the keys attended -- over its average launch span), `kernels` the
same for every projection and the attention; `traffic` is the HBM bytes per launch of that
kernel that rocprofv3's FETCH_SIZE + WRITE_SIZE counters read, scaled by the same counters on a
copy of known size (profiles/traffic_<workload>.txt, when present); `cpu_baseline` times the
oracle's CPU restatement of the reference decode step on the host for a bounded sample of the
same workload.
"""
import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "audiocraft.cpp_amd"))
sys.path.insert(0, ROOT)

WORKLOADS = {
    # name: shape, ggml weight type, prompt frames, continuation frames (max_gen_len = prompt + gen), seed, n_ctx
    "medium-q8": dict(shape="medium", wtype=8, prompt=500, gen=1500, seed=1, n_ctx=24,
                      desc="musicgen-medium-shaped LM, Q8_0, CFG 2 streams, 500-frame prompt + 1500-frame continuation"),
    "small-q8": dict(shape="small", wtype=8, prompt=250, gen=500, seed=0, n_ctx=12,
                     desc="musicgen-small-shaped LM, Q8_0, CFG 2 streams, 250-frame prompt + 500-frame continuation"),
    "small-f16": dict(shape="small", wtype=1, prompt=500, gen=1500, seed=0, n_ctx=12,
                      desc="musicgen-small-shaped LM, F16, CFG 2 streams, 500-frame prompt + 1500-frame continuation"),
    "large-q4": dict(shape="large", wtype=2, prompt=1500, gen=1500, seed=1, n_ctx=32,
                     desc="musicgen-large-shaped LM, Q4_0, CFG 2 streams, 1500-frame prompt + 1500-frame continuation"),
    # 8 independent requests in lockstep (16 streams), request r seeded 1 + r (memory, prompt,
    # sampling), rank-16 DoRA rows (alpha 16, strength 1) on every layer's qkv, ff.0 and ff.2
    "medium-q8-batch8-dora": dict(shape="medium", wtype=8, prompt=500, gen=1500, seed=1, n_ctx=24, requests=8,
                                  adapters=dict(rank=16, targets=("self.qkv", "ff.0", "ff.2"), dora=True),
                                  desc="musicgen-medium-shaped LM, Q8_0, 8 requests x CFG 2 streams (16 rows), "
                                       "rank-16 DoRA rows on qkv/ff.0/ff.2, 500-frame prompts + 1500-frame "
                                       "continuations"),
}
# The request server: 12 guided requests of mixed lengths submitted at once to 8 slots (request
# i: prompt 250 + (53 i mod 251) frames, continuation 500 + (97 i mod 501) frames, memory,
# prompt and sampling seeded 1 + i), against the same requests generated one after another.
SERVER = dict(shape="medium", wtype=8, slots=8, requests=12, n_ctx=24, seed=1,
              desc="musicgen-medium-shaped LM, Q8_0, 12 guided requests (prompts 250-500 frames, continuations "
                   "500-1000 frames) served by 8 slots vs one at a time")
BPW = {8: 34 / 32, 2: 18 / 32, 1: 2.0, 0: 4.0}
HBM_PEAK_GBS = 8000.0


def step_bytes(c, wbpw, n_seq, n_ctx, u, requests=1, adapter_bytes=0.0):
    """Algorithmic HBM bytes of one decode step attending u keys: weights at stored precision
    (cross.kv excluded: projected once per request) + adapter tensors (f32 A, B, magnitude and
    row norms, read once per step) + f32 LN params + f32 K/V read and write + each request's
    conditional-stream cross K/V + logits."""
    L, d, F, Q, C = c.layers, c.dim, c.ff_dim, c.n_q, c.card
    w = (L * (3 * d * d + d * d + d * d + d * d + 2 * d * F) + Q * C * d + Q * d) * wbpw + (6 * L + 2) * d * 4
    kv_read = 2 * L * d * u * n_seq * 4
    kv_write = 2 * L * d * n_seq * 4
    xkv = 2 * L * d * n_ctx * 4 * requests
    return w + adapter_bytes + kv_read + kv_write + xkv + Q * C * n_seq * 4


def unit_traffic(workload, kernel):
    """HBM bytes per launch of `kernel` from the committed counter summary, or None."""
    path = os.path.join(ROOT, "profiles", f"traffic_{workload.replace('-', '_')}.txt")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith(f"traffic_bytes_per_launch {kernel}:"):
                    return float(line.split(":", 1)[1])
    except OSError:
        return None
    return None


def hip_sync():
    lib = ctypes.CDLL("libamdhip64.so.7")
    rc = lib.hipDeviceSynchronize()
    if rc:
        raise RuntimeError(f"hipDeviceSynchronize failed: {rc}")


class CounterWindow:
    """roctxProfilerResume / Pause around the parts a counter run should see (rocprofv3
    --selected-regions collects only inside them): the calibration copy and the timed steps.
    Outside a profiler the calls do nothing."""

    def __init__(self, on):
        self.lib = None
        if on:
            self.lib = ctypes.CDLL("librocprofiler-sdk-roctx.so.1")
            self.lib.roctxProfilerPause.argtypes = [ctypes.c_uint64]
            self.lib.roctxProfilerResume.argtypes = [ctypes.c_uint64]
            self.lib.roctxProfilerPause(0)

    def __enter__(self):
        if self.lib:
            hip_sync()
            self.lib.roctxProfilerResume(0)
        return self

    def __exit__(self, *exc):
        if self.lib:
            hip_sync()
            self.lib.roctxProfilerPause(0)
        return False


def device_copy(mib):
    """One device-to-device copy of `mib` MiB: the known-size reference a counter run scales by."""
    lib = ctypes.CDLL("libamdhip64.so.7")
    n = int(mib) << 20
    a, b = ctypes.c_void_p(), ctypes.c_void_p()
    for p in (a, b):
        if lib.hipMalloc(ctypes.byref(p), ctypes.c_size_t(n)):
            raise RuntimeError("hipMalloc failed")
    # the buffers stay allocated until the process ends (a counter tool may still refer to them)
    if lib.hipMemset(a, 1, ctypes.c_size_t(n)) or lib.hipMemcpy(b, a, ctypes.c_size_t(n), 3):
        raise RuntimeError("device copy failed")
    hip_sync()


def cpu_baseline(w, model, t5, seconds, adapters=None):
    """The oracle (a CPU restatement of the reference's ggml-CPU decode step, including its
    per-step cross.kv projection) on the host, for about `seconds` of wall time: decode steps
    centred on the continuation's mean key count, as the GPU's timed steps are. The positions
    before them are not computed: the oracle's timing mode marks them as held by the cache
    (zero rows; a step's cost depends on how many keys it attends, not on their values), so the
    sample does not wait minutes for a prefill it does not time. For a batch workload it times
    one request: the reference serves requests one after another, so its aggregate rate is the
    one-request rate."""
    import numpy as np
    from oracle import cpu_ref as R
    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or os.cpu_count()
    R.set_threads(threads)
    rm = R.RefModel(model.config, model.tensors, adapters)
    c = model.config
    T = w["prompt"] + w["gen"]
    S = T + c.n_q
    start = w["prompt"] + 1
    mean_keys = (start + 1 + S - 1) // 2

    def run(n):
        # the first timed step attends mean_keys - n // 2 keys: a stand-in prompt of that length
        p = max(w["prompt"], mean_keys - n // 2 - 2)
        codes = np.zeros((c.n_q, p), np.int32)
        _, _, rep, _ = rm.generate(t5, codes, p, T, top_k=250, temperature=1.0, cfg_coef=3.0, seed=w["seed"],
                                   recompute_cross_kv=True, max_forwards=n + 1)
        return rep, p + 2

    R.lib().ref_set_timing_history(1)
    try:
        rep, _ = run(4)                                    # calibration
        per = max(rep.decode_seconds / 3, 1e-3)
        n = max(4, min(w["gen"], int(seconds / per)))
        rep, k0 = run(n)
    finally:
        R.lib().ref_set_timing_history(0)
    steps = rep.forwards - 1
    which = "one request of the batch (requests run one after another)" if w.get("requests", 1) > 1 else "same workload"
    return dict(value=round(steps / rep.decode_seconds, 3), unit="frames/s", cores=R.lib().ref_get_threads(),
                kind="port",
                sample=f"oracle CPU restatement of the reference ggml path, {which}: {steps} decode steps "
                       f"attending {k0}..{k0 + steps - 1} keys (centred on the continuation's mean, {mean_keys}) "
                       f"timed in {rep.decode_seconds:.1f} s; the positions before them held as zero cache "
                       f"rows, not computed")


def serve_bench(mgx):
    """Served throughput: every request submitted at t = 0 from its own thread to a server of
    8 slots; continuation frames of all requests over the wall time from the first submission
    to the last result (prefills included). The one-at-a-time figure runs the same requests
    through mgx_generate back to back -- the reference server's policy, on these kernels."""
    import threading
    w = SERVER
    model = mgx.SyntheticModel(w["shape"], w["wtype"], seed=w["seed"])
    c = model.config
    gm = mgx.Model(c, model.tensors)
    reqs = []
    for i in range(w["requests"]):
        P, G = 250 + (53 * i) % 251, 500 + (97 * i) % 501
        reqs.append(dict(P=P, G=G, t5=mgx.synth_memory(w["seed"] + i, w["n_ctx"]),
                         prompt=mgx.synth_codes(w["seed"] + i, c.n_q, P, c.card),
                         params=mgx.GenerateParams(P + G, 1, 1.0, 250, 3.0, w["seed"] + i)))
    frames = sum(r["G"] for r in reqs)
    srv = mgx.Server(gm, w["slots"], max(r["P"] + r["G"] for r in reqs), max_ctx=w["n_ctx"])
    # warm the graphs of every chunk count on one request, untimed
    r0 = reqs[-1]
    srv.generate(r0["t5"], r0["prompt"], r0["P"], r0["params"])
    before = srv.counters()
    out = [None] * len(reqs)

    def work(i):
        r = reqs[i]
        out[i] = srv.generate(r["t5"], r["prompt"], r["P"], r["params"])

    threads = [threading.Thread(target=work, args=(i,)) for i in range(len(reqs))]
    hip_sync()
    t0 = time.perf_counter()
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    served = time.perf_counter() - t0
    after = srv.counters()
    srv.close()
    steps = after["steps"] - before["steps"]
    occupancy = (after["slot_steps"] - before["slot_steps"]) / max(steps, 1)
    print(f"[bench] served {len(reqs)} requests in {served:.2f} s", file=sys.stderr, flush=True)
    hip_sync()
    t0 = time.perf_counter()
    for i, r in enumerate(reqs):
        codes = gm.generate(r["t5"], r["prompt"], r["P"], r["params"])[0]
        if not (codes == out[i][0]).all():
            raise RuntimeError(f"request {i}: served codes differ from generating alone")
    alone = time.perf_counter() - t0
    print(f"[bench] one at a time: {alone:.2f} s", file=sys.stderr, flush=True)
    print(json.dumps({
        "metric": "served LM frames/sec, MusicGen-medium Q8_0 CFG=2, mixed-length requests",
        "value": round(frames / served, 3), "unit": "frames/s", "n_gpus": 1, "steps": steps,
        "warmup": 1, "ms_per_step": round(1000.0 * served / max(steps, 1), 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8xq8_0+f32", "data": "synthetic (seeded random N(0,0.02) weights, N(0,1) memory, uniform "
                                          "prompt codes)",
        "config": {"workload": w["desc"], "requests": len(reqs), "slots": w["slots"], "layers": c.layers,
                   "dim": c.dim, "frames": frames, "prompt_frames": [r["P"] for r in reqs],
                   "continuation_frames": [r["G"] for r in reqs], "parallelism": "single GPU"},
        "served_seconds": round(served, 3),
        "one_at_a_time": {"value": round(frames / alone, 3), "unit": "frames/s", "seconds": round(alone, 3)},
        "speedup": round(alone / served, 3),
        "mean_occupancy": round(occupancy, 2),
    }), flush=True)


def t5_bench(mgx, reps, cpu):
    """The T5-base encoder (12 layers, 768 wide, F16 weights as tools/convert_t5.py writes them)
    over a 24-token prompt: encodes per second with the weights resident, against the oracle's
    CPU restatement of the same encode."""
    from mgx import synth
    m = synth.SyntheticT5("t5-base", 1, seed=1)
    ids = synth.synth_ids(1, 24, m.config.vocab)
    t5 = mgx.T5(m.config, m.tensors)
    for _ in range(3):
        t5.encode(ids)
    hip_sync()
    t0 = time.perf_counter()
    for _ in range(reps):
        t5.encode(ids)
    el = time.perf_counter() - t0
    out = {"metric": "T5-base encodes/sec, 24-token prompt, F16", "value": round(reps / el, 3), "unit": "encodes/s",
           "n_gpus": 1, "steps": reps, "warmup": 3, "ms_per_step": round(1000 * el / reps, 4),
           "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f16xf32",
           "data": "synthetic (seeded random weights and token ids)",
           "config": {"workload": "T5-base encoder, 12 layers, dim 768, 12 heads, FFN 3072, vocab 32128, F16, "
                                  "24 tokens, weights resident", "parallelism": "single GPU"}}
    if cpu:
        from oracle import cpu_ref as R
        threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or os.cpu_count()
        R.set_threads(threads)
        t0 = time.perf_counter()
        n = 0
        while time.perf_counter() - t0 < 10.0:
            R.t5_encode(m.config, m.tensors, ids)
            n += 1
        el = time.perf_counter() - t0
        out["cpu_baseline"] = {"value": round(n / el, 3), "unit": "encodes/s", "cores": R.lib().ref_get_threads(),
                               "kind": "port", "sample": f"oracle CPU restatement, {n} encodes of the same prompt "
                                                          f"({el:.1f} s)"}
    t5.close()
    print(json.dumps(out), flush=True)


def codec_bench(mgx, reps, cpu):
    """The EnCodec 32 kHz decoder over 1500 frames (30 s of audio): seconds of audio decoded per
    second, codes on the host to audio on the host, against the float64 oracle on a bounded
    sample."""
    from mgx import synth
    m = synth.SyntheticCodec("encodec-32k", seed=1)
    frames = 1500
    codes = m.codes(2, frames)
    k = mgx.Codec(m.config, m.tensors)
    k.decode(codes)
    hip_sync()
    t0 = time.perf_counter()
    for _ in range(reps):
        k.decode(codes)
    el = time.perf_counter() - t0
    audio_s = frames / m.config["frame_rate"]
    out = {"metric": "EnCodec 32 kHz decode, seconds of audio per second", "value": round(reps * audio_s / el, 3),
           "unit": "audio s/s", "n_gpus": 1, "steps": reps, "warmup": 1, "ms_per_step": round(1000 * el / reps, 3),
           "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
           "data": "synthetic (seeded random weights and codes)",
           "config": {"workload": "EnCodec 32 kHz decoder (ratios 8,5,4,4, 64 filters, 2-layer LSTM 1024, 4 x 2048 "
                                  "codebooks), 1500 frames = 30 s, codes to audio", "parallelism": "single GPU"}}
    if cpu:
        from oracle import codec_ref as K
        n = 100
        t0 = time.perf_counter()
        K.decode_codes(m.config, m.weights, codes[:, :n])
        el = time.perf_counter() - t0
        out["cpu_baseline"] = {"value": round(n / m.config["frame_rate"] / el, 4), "unit": "audio s/s",
                               "cores": os.cpu_count(), "kind": "port",
                               "sample": f"float64 numpy oracle (numpy's BLAS threads), {n} frames = "
                                         f"{n / m.config['frame_rate']:.0f} s of audio ({el:.1f} s)"}
    k.close()
    print(json.dumps(out), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1500)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--workload", default="medium-q8",
                    choices=sorted(WORKLOADS) + ["server-medium-q8", "t5-base", "encodec-decode"])
    ap.add_argument("--profile-steps", type=int, default=8,
                    help="decode steps whose launches are timed on the GPU clock after the timed run (untimed)")
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--prompt", type=int, default=None,
                    help="prompt frames override (counter runs: fewer untimed prefill dispatches)")
    ap.add_argument("--lead", type=int, default=None,
                    help="untimed decode steps before the warmup (default: centre the timed steps on the "
                         "continuation's middle; counter runs with a long --prompt pass 0)")
    ap.add_argument("--counter-window", action="store_true",
                    help="counter runs (rocprofv3 --selected-regions): collect only over the copy and the "
                         "timed steps")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="run one device-to-device copy of this many MiB first (counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (--gpus {args.gpus} requested). "
              "The decode step would shard by request, one process per GPU.", file=sys.stderr)
        sys.exit(2)
    import mgx
    if args.workload == "server-medium-q8":
        serve_bench(mgx)
        return
    if args.workload == "t5-base":
        t5_bench(mgx, args.steps if args.steps != 1500 else 200, not args.no_cpu)
        return
    if args.workload == "encodec-decode":
        codec_bench(mgx, args.steps if args.steps != 1500 else 5, not args.no_cpu)
        return
    w = dict(WORKLOADS[args.workload])
    if args.prompt is not None:
        w["prompt"] = args.prompt
    mgx.load()
    window = CounterWindow(args.counter_window)
    if args.copy_mib:
        with window:
            device_copy(args.copy_mib)
    t_build = time.time()
    model = mgx.SyntheticModel(w["shape"], w["wtype"], seed=w["seed"])
    c = model.config
    R = w.get("requests", 1)
    T = w["prompt"] + w["gen"]
    reqs = [dict(t5=mgx.synth_memory(w["seed"] + r, w["n_ctx"]),
                 prompt=mgx.synth_codes(w["seed"] + r, c.n_q, w["prompt"], c.card),
                 params=mgx.GenerateParams(T, 1, 1.0, 250, 3.0, w["seed"] + r)) for r in range(R)]
    t5, prompt = reqs[0]["t5"], reqs[0]["prompt"]
    gm = mgx.Model(c, model.tensors)
    adapters, adapter_bytes = None, 0.0
    if w.get("adapters"):
        adapters = mgx.synth_adapters(c, **w["adapters"])
        gm.set_adapters(adapters)
        # A, B, magnitude and the row norms, f32
        adapter_bytes = sum(4.0 * (a["A"].size + a["B"].size + 2 * a["B"].shape[0]) for a in adapters)
    print(f"[bench] {args.workload}: {model.nbytes() / 1e9:.2f} GB of weights built and uploaded in "
          f"{time.time() - t_build:.1f} s", file=sys.stderr, flush=True)
    S = T + c.n_q
    start = w["prompt"] + 1
    D = S - start - 1                                      # decode steps of one continuation

    def new_session():
        ss = mgx.Batch(gm, reqs, w["prompt"]) if R > 1 else mgx.Session(gm, t5, prompt, w["prompt"], reqs[0]["params"])
        hip_sync()
        tp = time.perf_counter()
        ss.step(1)                                         # prefill, outside the timed steps
        prefill_s.append(time.perf_counter() - tp)
        print(f"[bench] session prefilled ({start} tokens x {R} requests) in {prefill_s[-1]:.3f} s",
              file=sys.stderr, flush=True)
        return ss

    def keys_now(ss):
        return S - ss.remaining()                          # keys the next decode step attends

    timed = 0.0
    timed_steps = 0
    bytes_total = 0.0
    prefill_s = []
    segments = []
    # One continuation holds D decode steps whose attended keys grow from start + 1 to S - 1. A
    # run of fewer steps is centred on the continuation's middle, so its keys average what the
    # whole continuation's do: the steps before it run untimed (the last `warmup` of them just
    # before the timed ones).
    sess = new_session()
    lead = max(0, (D - args.steps) // 2 - args.warmup) if args.steps < D else 0
    if args.lead is not None:
        lead = max(0, args.lead)
    while lead > 0:
        lead -= sess.step(min(lead, 256))
    warm_left = args.warmup
    while timed_steps < args.steps:
        if sess.remaining() == 0:
            sess.close()
            sess = new_session()
        if warm_left > 0:
            warm_left -= sess.step(min(warm_left, sess.remaining()))
            continue
        n = min(args.steps - timed_steps, sess.remaining())
        u0 = keys_now(sess)
        with window:
            hip_sync()
            t0 = time.perf_counter()
            done = sess.step(n)
            hip_sync()
            timed += time.perf_counter() - t0
        for i in range(done):
            bytes_total += step_bytes(c, BPW[w["wtype"]], 2 * R, w["n_ctx"], u0 + i, R, adapter_bytes)
        segments.append([u0, u0 + done - 1])
        timed_steps += done
        print(f"[bench] timed {timed_steps}/{args.steps} steps, {timed:.2f} s", file=sys.stderr, flush=True)

    # Launch timing after the timed segment, untimed and outside the captured graphs: every
    # launch of `profile_steps` steps at the timed segment's middle keys (or right after it)
    # stamps its span on the GPU clock.
    kinds = {"gemv": 0, "attention": 1, "qkv": 2, "self.out": 3, "cross.q": 4, "cross.out": 5, "ff.0": 6,
             "ff.2": 7, "heads": 8, "cross-attention": 9}
    prof = {k: [0.0, 0.0, 0] for k in kinds}
    P = max(0, args.profile_steps)
    if P:
        mid = (segments[0][0] + segments[-1][1]) // 2
        if sess.remaining() < P:
            sess.close()
            sess = new_session()
            skip = max(0, mid - P // 2 - keys_now(sess))
            while skip > 0 and sess.remaining() > P:
                skip -= sess.step(min(skip, 256, sess.remaining() - P))
        prof_keys = keys_now(sess)
        sess.profile(1)
        sess.step(P)
        sess.profile(0)
        for k, kind in kinds.items():
            ms, by, nn = sess.profile_read(kind)
            prof[k] = [ms, by, nn]
    sess.close()

    def rate(k):
        ms, by, nn = prof[k]
        if nn == 0 or ms <= 0:
            return None
        return dict(achieved=round(by / (ms * 1e-3) / 1e9, 1), launches_timed=nn,
                    avg_launch_us=round(1000.0 * ms / nn, 3), bytes_per_launch=round(by / nn),
                    frac=round(by / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4))

    per_kernel = {k: rate(k) for k in kinds if k not in ("gemv",)}
    for k, v in per_kernel.items():
        if v is not None:
            v["traffic"] = unit_traffic(args.workload, k)
    timed_units = {k: v for k, v in per_kernel.items() if v is not None}
    # the dominant kernel: the largest share of a profiled step's GPU time
    dom = max(timed_units, key=lambda k: prof[k][0]) if timed_units else None
    wname = {8: "Q8_0", 2: "Q4_0", 1: "F16", 0: "F32"}[w["wtype"]]
    labels = {"qkv": f"k_gemv / k_gemv_mf self.qkv ({wname} weights, LayerNorm prologue, K/V append)",
              "self.out": f"self.out GEMV ({wname}, residual)", "cross.q": f"cross.q GEMV ({wname}, LayerNorm)",
              "cross.out": f"cross.out GEMV ({wname}, residual)",
              "ff.0": f"ff.0 GEMV ({wname} weights, LayerNorm prologue, GELU epilogue)",
              "ff.2": f"ff.2 GEMV ({wname}, residual)", "heads": f"output heads GEMV ({wname}, out_norm)",
              "attention": "self-attention (f32 K/V of the keys attended, every stream)",
              "cross-attention": "cross-attention (f32 K/V of each request's memory rows)"}
    fps = R * timed_steps / timed                          # frames of every request
    gemv_rate = rate("gemv")
    keys_mean = sum((a + b) * (b - a + 1) / 2 for a, b in segments) / max(timed_steps, 1)
    out = {
        "metric": "LM frames/sec & HBM GB/s, MusicGen-medium Q8_0 CFG=2, 30 s continuation"
        if args.workload == "medium-q8" else f"LM frames/sec & HBM GB/s, {args.workload}",
        "value": round(fps, 3),
        "unit": "frames/s",
        "n_gpus": 1,
        "steps": timed_steps,
        "warmup": args.warmup,
        "ms_per_step": round(1000.0 * timed / timed_steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {8: "int8xq8_0+f32", 2: "int8xq4_0+f32", 1: "f16+f32", 0: "f32"}[w["wtype"]],
        "data": "synthetic (seeded random N(0,0.02) weights, N(0,1) memory, uniform prompt codes)",
        "config": {"workload": w["desc"], "requests": R, "layers": c.layers, "dim": c.dim, "heads": c.heads,
                   "ff_dim": c.ff_dim, "weights": wname, "n_ctx": w["n_ctx"],
                   "prompt_frames": w["prompt"], "continuation_frames": w["gen"], "cfg_coef": 3.0, "top_k": 250,
                   "temperature": 1.0, "seed": w["seed"], "parallelism": "single GPU"},
        "timed_keys": {"segments": segments, "mean": round(keys_mean, 1),
                       "continuation_mean": round((start + 1 + S - 1) / 2, 1)},
        "hbm_gbs_step": round(bytes_total / timed / 1e9, 1),
        "roofline_frac_step": round(bytes_total / timed / 1e9 / HBM_PEAK_GBS, 4),
        "roofline": None if dom is None else {
            "bound": "hbm", "achieved": timed_units[dom]["achieved"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": timed_units[dom]["frac"], "traffic": unit_traffic(args.workload, dom),
            "kernel": labels[dom], "launches_timed": timed_units[dom]["launches_timed"],
            "avg_launch_us": timed_units[dom]["avg_launch_us"],
            "bytes_per_launch": timed_units[dom]["bytes_per_launch"], "profiled_keys": prof_keys},
        "gemv_family": gemv_rate,
        "kernels": per_kernel,
        # the prompt's prefill (the loop's first forward, start tokens), outside `value`
        "prefill_ms": round(1000.0 * min(prefill_s), 2) if prefill_s else None,
    }
    if not args.no_cpu:
        try:
            out["cpu_baseline"] = cpu_baseline(w, model, t5, args.cpu_seconds, adapters)
        except Exception as e:  # the GPU figure stands without it
            out["cpu_baseline"] = {"error": str(e)}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
