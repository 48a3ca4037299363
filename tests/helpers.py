"""Shared fixtures-in-code for the tests: seeded synthetic models and their oracle twins."""
import functools

import numpy as np

from mgx import synth
from oracle import cpu_ref as R


@functools.lru_cache(maxsize=None)
def model(shape, wtype, seed=0, **over):
    return synth.SyntheticModel(shape, wtype, seed=seed, **over)


@functools.lru_cache(maxsize=None)
def ref_model(shape, wtype, seed=0):
    m = model(shape, wtype, seed)
    return R.RefModel(m.config, m.tensors)


def memory(seed, n_ctx):
    return synth.synth_memory(seed, n_ctx)


def codes(seed, n_q, length, card):
    return synth.synth_codes(seed, n_q, length, card)


def first_diff(a, b):
    a = np.asarray(a).reshape(-1)
    b = np.asarray(b).reshape(-1)
    idx = np.nonzero(a != b)[0]
    return None if idx.size == 0 else int(idx[0])
