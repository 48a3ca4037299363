"""The oracle's numeric primitives against closed forms and independent implementations:
exp / erf against 200-bit mpmath, expf / erff against glibc, fp16 conversion against numpy,
LayerNorm, the sinusoid and attention against float64 numpy, the Q8_0 quantizer against its
defining properties."""
import ctypes as C
import ctypes.util
import math

import mpmath
import numpy as np
import pytest

from oracle import cpu_ref as R

L = R.lib()
libm = C.CDLL(ctypes.util.find_library("m"))
libm.expf.restype = C.c_float
libm.expf.argtypes = [C.c_float]
libm.erff.restype = C.c_float
libm.erff.argtypes = [C.c_float]
mpmath.mp.prec = 200


def ulps(got, exact):
    e = float(exact)
    return abs(mpmath.mpf(got) - exact) / math.ulp(e) if e != 0 else abs(got)


def test_exp_within_one_ulp():
    rs = np.random.default_rng(0)
    xs = np.concatenate([rs.uniform(-745, 709, 3000), rs.uniform(-2, 2, 3000), [0.0, 1.0, -1.0, 0.5, 709.7]])
    worst = max(ulps(L.ref_exp(float(x)), mpmath.exp(float(x))) for x in xs)
    assert worst <= 1.0
    assert L.ref_exp(-800.0) == 0.0 and math.isinf(L.ref_exp(710.0)) and math.isnan(L.ref_exp(float("nan")))


def test_erf_accuracy_and_odd():
    """The two-interpolant erf: relative error below 4e-15 for |x| < 1 (erf ~ x there), absolute
    error below 2e-12 on [1, 4), exactly +-1 beyond, odd."""
    rs = np.random.default_rng(1)
    xs = np.concatenate([rs.uniform(-7, 7, 4000), rs.uniform(-1, 1, 2000),
                         [1e-300, 1e-8, 0.9999999, 1.0, 1.0000001, 2.5, 3.9999999, 4.0, 6.0]])
    for x in xs:
        got, want = L.ref_erf(float(x)), mpmath.erf(float(x))
        if abs(x) < 1:
            assert abs(mpmath.mpf(got) - want) <= 4e-15 * abs(want), float(x)
        elif abs(x) < 4:
            assert abs(mpmath.mpf(got) - want) <= 2e-12, float(x)
        else:
            assert got == math.copysign(1.0, x)
    for x in xs[:200]:
        assert L.ref_erf(float(-x)) == -L.ref_erf(float(x))
    assert L.ref_erf(0.0) == 0.0


def test_expf_erff_rounding():
    """(float) of the double routines: expf is the correctly rounded value on every sample
    (checked against 200-bit mpmath); erff is within one ulp of the true erf everywhere and the
    correctly rounded value on all but a few in 10^4 samples (its double erf is accurate to
    1.3e-12 absolute, so only values that close to a rounding midpoint can round the other
    way); glibc's own expf / erff, which ggml's scalar path calls, agree to 1 ulp."""
    rs = np.random.default_rng(2)
    xs = np.concatenate([rs.uniform(-88, 88, 6000), rs.normal(0, 2, 6000)]).astype(np.float32)
    for x in xs:
        got = np.float32(L.ref_expf(float(x)))
        assert got == np.float32(float(mpmath.exp(float(x)))), float(x)
        g = np.float32(libm.expf(float(x)))
        assert abs(int(got.view(np.int32)) - int(g.view(np.int32))) <= 1
    off = 0
    ys = np.concatenate([rs.normal(0, 2, 6000), rs.uniform(-4.5, 4.5, 6000)]).astype(np.float32)
    for y in ys:
        got = np.float32(L.ref_erff(float(y)))
        exact = np.float32(float(mpmath.erf(float(y))))
        assert abs(int(got.view(np.int32)) - int(exact.view(np.int32))) <= 1, float(y)
        off += got != exact
        g = np.float32(libm.erff(float(y)))
        assert abs(int(got.view(np.int32)) - int(g.view(np.int32))) <= 1
    assert off <= 6, off


def test_gelu_erf_closed_form():
    for x in np.linspace(-8, 8, 801).astype(np.float32):
        want = 0.5 * float(x) * (1.0 + math.erf(float(x) / math.sqrt(2.0)))
        assert abs(L.ref_gelu_erf(float(x)) - want) <= 2e-7 * max(1.0, abs(want))
    assert L.ref_gelu_erf(0.0) == 0.0


def test_fp16_conversions_match_numpy():
    rs = np.random.default_rng(3)
    xs = np.concatenate([rs.normal(0, 1, 20000), rs.normal(0, 1e-5, 5000), rs.normal(0, 3e4, 2000),
                         [65504.0, 65520.0, 65519.99, 6.1035156e-05, 5.96e-08, 2.98e-08, 0.0, -0.0, 1e-9]]).astype(np.float32)
    got = np.array([L.ref_fp32_to_fp16(float(x)) for x in xs], np.uint16)
    want = xs.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    hs = np.arange(0, 65536, 7, dtype=np.uint16)
    hs = hs[(hs & 0x7c00) != 0x7c00]
    back = np.array([L.ref_fp16_to_fp32(int(h)) for h in hs], np.float32)
    assert np.array_equal(back, hs.view(np.float16).astype(np.float32))


def test_q8_0_quantizer_properties():
    rs = np.random.default_rng(4)
    x = rs.normal(0, 1, 32 * 64).astype(np.float32)
    x[:32] = 0.0                                          # an all-zero block
    out = np.zeros(34 * 64, np.uint8)
    L.ref_quantize_q8_0(R.ptr(x), x.size, R.ptr(out))
    blocks = out.reshape(64, 34)
    d = blocks[:, :2].copy().view(np.float16).astype(np.float32).reshape(-1)
    q = blocks[:, 2:].view(np.int8).astype(np.float32)
    assert d[0] == 0 and (q[0] == 0).all()
    xb = x.reshape(64, 32)
    amax = np.abs(xb).max(axis=1)
    np.testing.assert_allclose(d[1:], (amax[1:] / 127).astype(np.float16).astype(np.float32))
    assert (np.abs(q[1:]).max(axis=1) == 127).all()
    err = np.abs(q * d[:, None] - xb)
    assert (err[1:] <= d[1:, None] * 0.5 + 1e-3 * d[1:, None] + np.abs(xb[1:]) * 2e-3).all()


def test_synth_packer_agrees_with_oracle_quantizer():
    from mgx import synth
    rs = np.random.default_rng(5)
    x = rs.normal(0, 0.02, (8, 96)).astype(np.float32)
    a = synth.pack(8, x)
    b = np.zeros_like(a)
    L.ref_quantize_q8_0(R.ptr(x), x.size, R.ptr(b))
    assert np.array_equal(a, b)


def test_layer_norm_against_float64():
    rs = np.random.default_rng(6)
    for n in (128, 1024, 1536, 2048, 768):
        x = rs.normal(0.3, 2.0, n).astype(np.float32)
        w = rs.normal(1, 0.1, n).astype(np.float32)
        b = rs.normal(0, 0.1, n).astype(np.float32)
        y = np.zeros(n, np.float32)
        L.ref_layer_norm(R.ptr(x), n, R.ptr(w), R.ptr(b), 1e-5, R.ptr(y))
        xd = x.astype(np.float64)
        want = (xd - xd.mean()) / np.sqrt(xd.var() + 1e-5) * w + b
        np.testing.assert_allclose(y, want, atol=2e-6, rtol=2e-6)


def test_sin_positions_formula():
    """lm.h:102-116: cos/sin(pos / max_period^(i / (half-1)))."""
    dim, den, n = 64, 31, 40
    out = np.zeros((n, dim), np.float32)
    L.ref_sin_positions(100, n, dim, den, 10000.0, R.ptr(out))
    i = np.arange(dim // 2)
    pos = np.arange(100, 100 + n)[:, None].astype(np.float64)
    phase = pos / np.power(10000.0, i / den)
    np.testing.assert_allclose(out, np.concatenate([np.cos(phase), np.sin(phase)], axis=1).astype(np.float32),
                               atol=1e-7, rtol=0)
    # the last frequency is exactly 1/max_period (the half-1 denominator)
    assert out[0, dim - 1] == np.float32(np.sin(100 / 10000.0)) and out[0, dim // 2 - 1] == np.float32(np.cos(0.01))


def test_attention_against_dense_float64():
    """sdpa_vt on the transposed cache = dense softmax attention (nn.h:186-191), with chunks
    whose maxima differ widely (a block of keys aligned with q) so the per-chunk rescaling
    carries real weight."""
    rs = np.random.default_rng(7)
    for u in (1, 7, 64, 65, 256, 257, 1000, 3003, 4096):
        hd, cap = 64, u + 5
        q = rs.normal(0, 1, hd).astype(np.float32)
        K = rs.normal(0, 1, (u, hd)).astype(np.float32)
        if u > 300:
            K[260:290] += (3.0 * q / np.linalg.norm(q)).astype(np.float32)
        VT = rs.normal(0, 1, (hd, cap)).astype(np.float32)
        out = np.zeros(hd, np.float32)
        L.ref_attend(R.ptr(q), hd, u, R.ptr(K), R.ptr(VT), cap, None, 0.125, R.ptr(out))
        s = K.astype(np.float64) @ q.astype(np.float64) * 0.125
        p = np.exp(s - s.max())
        p /= p.sum()
        want = VT[:, :u].astype(np.float64) @ p
        np.testing.assert_allclose(out, want, atol=2e-6, rtol=1e-5)
        if u > 300:
            # the plausible combine mistakes (chunks not rescaled by exp(m_c - M), or the
            # total taken over the last chunk only) miss this tolerance by far
            nch = (u + 63) // 64
            m = np.array([s[64 * c:64 * c + 64].max() for c in range(nch)])
            e = [np.exp(s[64 * c:64 * c + 64] - m[c]) for c in range(nch)]
            o = np.array([VT[:, 64 * c:64 * c + len(e[c])].astype(np.float64) @ e[c] for c in range(nch)])
            S = np.array([x.sum() for x in e])
            unscaled = o.sum(0) / S.sum()
            w = np.exp(m - m.max())
            right = (o * w[:, None]).sum(0) / (S * w).sum()
            np.testing.assert_allclose(right, want, atol=1e-12)
            assert np.abs(unscaled - want).max() > 100 * 2e-6
            assert np.abs((o * w[:, None]).sum(0) / S[-1] - want).max() > 100 * 2e-6


def test_masked_attention_equals_shorter_history():
    """A causal mask only adds exact zeros: masking keys >= m equals attending m keys."""
    rs = np.random.default_rng(8)
    hd, u, cap = 64, 600, 600
    q = rs.normal(0, 1, hd).astype(np.float32)
    K = rs.normal(0, 1, (u, hd)).astype(np.float32)
    VT = rs.normal(0, 1, (hd, cap)).astype(np.float32)
    for m in (1, 255, 256, 300, 599):
        mask = np.where(np.arange(u) < m, 0.0, -np.inf).astype(np.float32)
        a = np.zeros(hd, np.float32)
        b = np.zeros(hd, np.float32)
        L.ref_attend(R.ptr(q), hd, u, R.ptr(K), R.ptr(VT), cap, R.ptr(mask), 0.125, R.ptr(a))
        L.ref_attend(R.ptr(q), hd, m, R.ptr(K), R.ptr(VT), cap, None, 0.125, R.ptr(b))
        assert np.array_equal(a, b)
