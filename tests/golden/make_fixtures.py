#!/usr/bin/env python3
"""Writes the oracle's full-length generation fixtures (tests/golden/<case>.npz).

Each case is one of the benchmark configurations, run end to end through the oracle's
restatement of mg_generate (prefill of the prompt with the causal mask, then every decode
step, CFG mix, top-k sampling with the reference's mt19937 stream). A fixture holds the codes
[n_q][T], the first mixed logits [n_q][card], a CRC32 per step of the mixed logits (to name the
first step where two runs part), and checksums of the inputs so a change in the synthetic
generator is caught instead of silently compared against.

Usage: python tests/golden/make_fixtures.py c1 [c2 ...]   (runs minutes to tens of minutes)
"""
import hashlib
import os
import sys
import time
import zlib

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "audiocraft.cpp_amd"))

from mgx import synth  # noqa: E402
from oracle import cpu_ref as R  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))

# The four single-request workloads at full length: small Q8_0 p250+c500, small F16 p500+c1500,
# medium Q8_0 p500+c1500, large Q4_0 p1500+c1500; and the batched serving workload: 8 guided
# medium Q8_0 requests (request r seeded 1 + r: memory, prompt, sampling) with rank-16 DoRA rows
# on every layer's qkv, ff.0 and ff.2, each request generated alone by the oracle.
CASES = {
    "c1_small_q8": dict(shape="small", wtype=8, prompt=250, gen=500, seed=0, sampling=True, top_k=250),
    "c1_small_q8_greedy": dict(shape="small", wtype=8, prompt=250, gen=500, seed=0, sampling=False, top_k=250),
    "c2_small_f16_topk1": dict(shape="small", wtype=1, prompt=500, gen=1500, seed=0, sampling=True, top_k=1),
    "c3_medium_q8": dict(shape="medium", wtype=8, prompt=500, gen=1500, seed=1, sampling=True, top_k=250),
    "c4_large_q4": dict(shape="large", wtype=2, prompt=1500, gen=1500, seed=1, sampling=True, top_k=250),
    "c5_medium_q8_batch8_dora": dict(shape="medium", wtype=8, prompt=500, gen=1500, seed=1, sampling=True, top_k=250,
                                     requests=8, adapters=dict(rank=16, targets=("self.qkv", "ff.0", "ff.2"),
                                                               dora=True)),
}
ALIASES = {"c1": ["c1_small_q8", "c1_small_q8_greedy"], "c2": ["c2_small_f16_topk1"], "c3": ["c3_medium_q8"],
           "c4": ["c4_large_q4"], "c5": ["c5_medium_q8_batch8_dora"]}


def model_digest(model):
    h = hashlib.sha256()
    for name, ttype, ne0, ne1, data in model.tensors:
        h.update(name.encode())
        h.update(np.array([ttype, ne0, ne1], np.int64).tobytes())
        h.update(data.tobytes())
    return h.hexdigest()


def inputs(case):
    m = synth.SyntheticModel(case["shape"], case["wtype"], seed=case["seed"])
    n_ctx = synth.SHAPES[case["shape"]]["n_ctx"]
    t5 = synth.synth_memory(case["seed"], n_ctx)
    prompt = synth.synth_codes(case["seed"], m.config.n_q, case["prompt"], m.config.card)
    return m, t5, prompt


def batch_inputs(case):
    """The model, its adapters and request r's (memory, prompt, seed), r = 0 .. requests - 1."""
    m = synth.SyntheticModel(case["shape"], case["wtype"], seed=case["seed"])
    ads = synth.synth_adapters(m.config, **case["adapters"])
    n_ctx = synth.SHAPES[case["shape"]]["n_ctx"]
    reqs = [(synth.synth_memory(case["seed"] + r, n_ctx),
             synth.synth_codes(case["seed"] + r, m.config.n_q, case["prompt"], m.config.card), case["seed"] + r)
            for r in range(case["requests"])]
    return m, ads, reqs


def adapter_digest(ads):
    h = hashlib.sha256()
    for a in ads:
        h.update(a["target"].encode())
        for k in ("A", "B", "magnitude"):
            if a.get(k) is not None:
                h.update(a[k].tobytes())
    return h.hexdigest()


def make_batch(name):
    case = CASES[name]
    t0 = time.time()
    m, ads, reqs = batch_inputs(case)
    rm = R.RefModel(m.config, m.tensors, ads)
    T = case["prompt"] + case["gen"]
    codes, firsts, crcs, t5c, pc = [], [], [], [], []
    for r, (t5, prompt, seed) in enumerate(reqs):
        c, f, rep, steps = rm.generate(t5, prompt, case["prompt"], T, use_sampling=case["sampling"], temperature=1.0,
                                       top_k=case["top_k"], cfg_coef=3.0, seed=seed, step_logits=True)
        codes.append(c)
        firsts.append(f)
        crcs.append([zlib.crc32(steps[i].tobytes()) for i in range(steps.shape[0])])
        t5c.append(zlib.crc32(t5.tobytes()))
        pc.append(zlib.crc32(prompt.tobytes()))
        print(f"{name} request {r}: {rep.forwards} forwards, prefill {rep.prefill_seconds:.1f} s, "
              f"decode {rep.decode_seconds:.1f} s", flush=True)
    np.savez_compressed(os.path.join(HERE, name + ".npz"), codes=np.stack(codes), first_logits=np.stack(firsts),
                        step_crc=np.array(crcs, np.uint32),
                        model_sha256=np.frombuffer(bytes.fromhex(model_digest(m)), np.uint8),
                        adapter_sha256=np.frombuffer(bytes.fromhex(adapter_digest(ads)), np.uint8),
                        t5_crc=np.array(t5c, np.uint32), prompt_crc=np.array(pc, np.uint32),
                        convention=np.int32(R.lib().ref_convention()))
    print(f"{name}: total {time.time() - t0:.1f} s", flush=True)


def make(name):
    case = CASES[name]
    if case.get("requests"):
        make_batch(name)
        return
    t0 = time.time()
    m, t5, prompt = inputs(case)
    rm = R.RefModel(m.config, m.tensors)
    T = case["prompt"] + case["gen"]
    codes, first, rep, steps = rm.generate(t5, prompt, case["prompt"], T, use_sampling=case["sampling"],
                                           temperature=1.0, top_k=case["top_k"], cfg_coef=3.0, seed=case["seed"],
                                           step_logits=True)
    crc = np.array([zlib.crc32(steps[i].tobytes()) for i in range(steps.shape[0])], np.uint32)
    np.savez_compressed(os.path.join(HERE, name + ".npz"), codes=codes, first_logits=first, step_crc=crc,
                        model_sha256=np.frombuffer(bytes.fromhex(model_digest(m)), np.uint8),
                        t5_crc=np.uint32(zlib.crc32(t5.tobytes())), prompt_crc=np.uint32(zlib.crc32(prompt.tobytes())),
                        prefill_seconds=rep.prefill_seconds, decode_seconds=rep.decode_seconds,
                        convention=np.int32(R.lib().ref_convention()))
    print(f"{name}: {rep.forwards} forwards, prefill {rep.prefill_seconds:.1f} s, decode {rep.decode_seconds:.1f} s, "
          f"total {time.time() - t0:.1f} s", flush=True)


if __name__ == "__main__":
    todo = []
    for a in sys.argv[1:] or ["c1"]:
        todo += ALIASES.get(a, [a])
    for name in todo:
        make(name)
