"""mgx_t5_encode_static -- the T5 encode with its working memory in a file-scope device array,
allocating nothing -- against mgx_t5_encode on the same encoder, bit for bit, through the C
ABI: two calls in a row (the second shorter, so it runs over what the first left in the
shared array), then the size check."""
import ctypes as C

import numpy as np
import pytest

from mgx import synth

pytestmark = pytest.mark.gpu


def encode_static(lib, t5, ids):
    ids = np.ascontiguousarray(ids, np.int32)
    out = np.zeros((ids.size, t5.config.dim), np.float32)
    fn = lib.mgx_t5_encode_static
    fn.argtypes = [C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p]
    fn.restype = C.c_int
    rc = fn(t5.handle, ids.ctypes.data, ids.size, out.ctypes.data)
    return rc, out


@pytest.mark.parametrize("shape,wtype", [("t5-mini", 1), ("t5-tiny", 8), ("t5-tiny", 2)])
def test_static_encode_equals_encode(shape, wtype):
    import mgx
    lib = mgx.load()
    print(f"static T5 encode {shape} wtype={wtype}: 200 then 37 tokens", flush=True)
    m = synth.SyntheticT5(shape, wtype, seed=11)
    t5 = mgx.T5(m.config, m.tensors)
    for n, seed in ((200, 1), (37, 2)):
        ids = synth.synth_ids(seed, n, m.config.vocab)
        rc, got = encode_static(lib, t5, ids)
        assert rc == 0, lib.mgx_last_error()
        want = t5.encode(ids)
        assert np.array_equal(got, want), f"{n} tokens: max {np.abs(got - want).max()}"
    t5.close()


def test_static_encode_checks():
    import mgx
    lib = mgx.load()
    lib.mgx_last_error.restype = C.c_char_p
    m = synth.SyntheticT5("t5-tiny", 1, seed=12)
    t5 = mgx.T5(m.config, m.tensors)
    rc, _ = encode_static(lib, t5, np.zeros(257, np.int32))
    assert rc == -1 and b"1 to 256 tokens" in lib.mgx_last_error()
    rc, _ = encode_static(lib, t5, np.full(3, m.config.vocab, np.int32))
    assert rc == -1 and b"out of range" in lib.mgx_last_error()
    # an encoder whose 256-token encode needs more than the 32 MiB array
    big = synth.SyntheticT5(dict(dim=2048, layers=1, heads=32, intermediate=8192, vocab=64), 8, seed=13)
    tb = mgx.T5(big.config, big.tensors)
    rc, _ = encode_static(lib, tb, synth.synth_ids(3, 256, 64))
    assert rc == -1 and b"MiB of scratch" in lib.mgx_last_error()
    rc, got = encode_static(lib, tb, synth.synth_ids(4, 16, 64))
    assert rc == 0, lib.mgx_last_error()
    assert np.array_equal(got, tb.encode(synth.synth_ids(4, 16, 64)))
    tb.close()
    t5.close()
