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
# medium Q8_0 p500+c1500, large Q4_0 p1500+c1500 (the batched DoRA workload is checked against
# the oracle live).
CASES = {
    "c1_small_q8": dict(shape="small", wtype=8, prompt=250, gen=500, seed=0, sampling=True, top_k=250),
    "c1_small_q8_greedy": dict(shape="small", wtype=8, prompt=250, gen=500, seed=0, sampling=False, top_k=250),
    "c2_small_f16_topk1": dict(shape="small", wtype=1, prompt=500, gen=1500, seed=0, sampling=True, top_k=1),
    "c3_medium_q8": dict(shape="medium", wtype=8, prompt=500, gen=1500, seed=1, sampling=True, top_k=250),
    "c4_large_q4": dict(shape="large", wtype=2, prompt=1500, gen=1500, seed=1, sampling=True, top_k=250),
}
ALIASES = {"c1": ["c1_small_q8", "c1_small_q8_greedy"], "c2": ["c2_small_f16_topk1"], "c3": ["c3_medium_q8"],
           "c4": ["c4_large_q4"]}


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


def make(name):
    case = CASES[name]
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
