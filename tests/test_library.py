"""The C-ABI library on the CPU: it loads, exports every entry point include/mgx.h declares,
and its host-side checks reject bad input before touching a device."""
import ctypes as C
import os
import re

import numpy as np
import pytest

import mgx
from mgx import synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    text = open(os.path.join(ROOT, "include", "mgx.h")).read()
    return sorted(set(re.findall(r"\b(mgx_\w+)\s*\(", text)))


def test_library_exports_every_declared_entry_point():
    lib = mgx.load()
    names = declared()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing
    assert set(mgx.lib.EXPORTS) <= set(names)


def test_use_guidance_rule():
    """pipeline.h:41-43 and tests/conditioner_test.cpp:52-65."""
    assert mgx.use_guidance(3.0, False) and not mgx.use_guidance(3.0, True)
    assert not mgx.use_guidance(0.0, False) and not mgx.use_guidance(0.0, True)


@pytest.mark.parametrize("field,value,msg", [
    ("dim", 100, "heads"), ("special_token_id", 7, "special_token_id"), ("head_dim", 32, "head_dim"),
    ("card", 4096, "card"), ("n_q", 9, "n_q"),
])
def test_model_config_rejected_before_any_device_call(field, value, msg):
    m = synth.SyntheticModel("tiny", 8, seed=1)
    cfg = synth.make_config("tiny")
    setattr(cfg, field, value)
    if field == "head_dim":
        cfg.heads = cfg.dim // 32
    with pytest.raises(mgx.MgxError, match=msg):
        mgx.Model(cfg, m.tensors)


def test_missing_and_misshapen_tensors_rejected():
    m = synth.SyntheticModel("tiny", 8, seed=1)
    with pytest.raises(mgx.MgxError, match="missing tensor lm.0.ff.2.weight"):
        mgx.Model(m.config, [t for t in m.tensors if t[0] != "lm.0.ff.2.weight"])
    bad = [(n, ty, e0, e1 + (1 if n == "lm.1.self.out.weight" else 0), d) for n, ty, e0, e1, d in m.tensors]
    with pytest.raises(mgx.MgxError, match="bad shape for lm.1.self.out.weight"):
        mgx.Model(m.config, bad)


def test_synthetic_weights_are_deterministic():
    a = synth.SyntheticModel("tiny", 8, seed=5)
    b = synth.SyntheticModel("tiny", 8, seed=5)
    c = synth.SyntheticModel("tiny", 8, seed=6)
    assert all(np.array_equal(x[4], y[4]) for x, y in zip(a.tensors, b.tensors))
    assert not np.array_equal(a.tensor("lm.0.self.qkv.weight")[4], c.tensor("lm.0.self.qkv.weight")[4])
    w = synth.SyntheticModel("tiny", 0, seed=5).tensor("lm.0.ff.0.weight")[4].view(np.float32)
    assert abs(w.std() - 0.02) < 0.002 and abs(w.mean()) < 0.002
    assert synth.synth_codes(1, 4, 100, 2048).max() < 2048
