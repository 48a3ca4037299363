#!/usr/bin/env python3
"""Copies the golden vectors that the reference's own unit tests hold -- as data -- into
tests/golden/*.json: the softmax / top-k / argmax fixtures of tests/sampling_test.cpp
(generated there by tests/gen_sampling_fixture.py from audiocraft's sample_top_k) and the
delay-pattern fixtures of tests/pattern_test.cpp (from audiocraft's DelayedPatternProvider),
the T5 relative-position buckets of tests/t5_bucket_test.cpp (from transformers'
T5Attention._relative_position_bucket, bidirectional, 32 buckets, max distance 128), the
torch.nn.LSTM vectors of tests/lstm_test.cpp (tests/gen_lstm_fixture.py) and the residual
vector quantizer vectors of tests/codec_test.cpp (transformers' EncodecResidualVectorQuantizer,
tests/gen_codec_fixture.py).

Reads the reference tree as text (default /root/reference); run once, outputs committed."""
import json
import os
import re
import sys

REF = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
HERE = os.path.dirname(os.path.abspath(__file__))


def arrays(text, ctype):
    out = {}
    for m in re.finditer(r"static const %s (\w+)\[\] = \{([^}]*)\};" % ctype, text):
        vals = [v.strip().rstrip("f") for v in m.group(2).replace("\n", " ").split(",") if v.strip()]
        out[m.group(1)] = [float(v) if ctype == "float" else int(v) for v in vals]
    return out


def consts(text):
    out = {}
    for m in re.finditer(r"constexpr (?:int|float) ([^;]+);", text):
        for part in m.group(1).split(","):
            k, v = part.split("=")
            out[k.strip()] = float(v.strip().rstrip("f"))
    return out


def sampling():
    text = open(os.path.join(REF, "tests", "sampling_test.cpp")).read()
    fa, cs = arrays(text, "float"), consts(text)
    cases = {}
    for tag in ("PLAIN", "HOT", "COLD", "WIDE", "TIED"):
        cases[tag] = dict(n=int(cs[f"{tag}_N"]), k=int(cs[f"{tag}_K"]), survivors=int(cs[f"{tag}_SURVIVORS"]),
                          temperature=cs[f"{tag}_TEMPERATURE"], argmax=int(cs[f"{tag}_ARGMAX"]),
                          logits=fa[f"{tag}_logits"], softmax=fa[f"{tag}_softmax"], filtered=fa[f"{tag}_filtered"])
    return {"source": "tests/sampling_test.cpp:81-192", "cases": cases}


def pattern():
    text = open(os.path.join(REF, "tests", "pattern_test.cpp")).read()
    ia, cs = arrays(text, "int32_t"), consts(text)
    cases = {}
    for tag in ("MG", "ONE", "THREE"):
        cases[tag] = dict(n_q=int(cs[f"{tag}_NQ"]), timesteps=int(cs[f"{tag}_T"]), steps=int(cs[f"{tag}_S"]),
                          special=int(cs[f"{tag}_SPECIAL"]), codes=ia[f"{tag}_codes"], sequence=ia[f"{tag}_sequence"],
                          mask=ia[f"{tag}_mask"], reverted=ia[f"{tag}_reverted"], first_step=ia[f"{tag}_first_step"])
    return {"source": "tests/pattern_test.cpp:90-146", "cases": cases}


def t5_buckets():
    text = open(os.path.join(REF, "tests", "t5_bucket_test.cpp")).read()
    body = text[text.index("static const Case cases[] = {"):]
    body = body[:body.index("};")]
    pairs = [(int(a), int(b)) for a, b in re.findall(r"\{(-?\d+),\s*(-?\d+)\}", body)]
    return {"source": "tests/t5_bucket_test.cpp:26-31", "num_buckets": 32, "max_distance": 128,
            "cases": [{"relative_position": a, "bucket": b} for a, b in pairs]}


def lstm():
    text = open(os.path.join(REF, "tests", "lstm_test.cpp")).read()
    fa = arrays(text, "float")
    m = re.search(r"constexpr int H = (\d+), T = (\d+), L = (\d+);", text)
    H, T, L = (int(v) for v in m.groups())
    return {"source": "tests/lstm_test.cpp:57-111 (torch.nn.LSTM, tests/gen_lstm_fixture.py)", "hidden": H,
            "frames": T, "layers": L, "arrays": fa}


def rvq():
    text = open(os.path.join(REF, "tests", "codec_test.cpp")).read()
    fa, ia = arrays(text, "float"), arrays(text, "int32_t")
    m = re.search(r"constexpr int RVQ_NQ = (\d+), RVQ_BINS = (\d+), RVQ_DIM = (\d+), RVQ_FRAMES = (\d+);", text)
    nq, bins, dim, frames = (int(v) for v in m.groups())
    return {"source": "tests/codec_test.cpp:82-181 (EncodecResidualVectorQuantizer, tests/gen_codec_fixture.py)",
            "n_q": nq, "bins": bins, "dim": dim, "frames": frames, "embed": fa["rvq_embed"],
            "latent": fa["rvq_latent"], "codes": ia["rvq_codes"], "quantized": fa["rvq_quantized"]}


if __name__ == "__main__":
    for name, fn in (("sampling_cases.json", sampling), ("pattern_cases.json", pattern),
                     ("t5_bucket_cases.json", t5_buckets), ("lstm_cases.json", lstm), ("rvq_cases.json", rvq)):
        with open(os.path.join(HERE, name), "w") as f:
            json.dump(fn(), f, indent=1)
        print("wrote", name)
