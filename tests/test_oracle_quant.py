"""The oracle's quantized and half-precision LM forward against an independent float64 model.

The oracle (oracle/cpu_ref.c) multiplies Q8_0 / Q4_0 weights against activations quantized to
Q8_0 per 32-element block with integer block dots, and F16 weights against fp16-rounded
activations (ggml's vec_dot_type conversion; the reference reaches it through every
ggml_mul_mat of src/mg/lm.h:152-259 and src/ac/lora.h:53). This file restates only the
arithmetic those conventions fix, with its own code:

  * weights decoded from the ggml block bytes in numpy: Q8_0 {fp16 d; int8 q[32]} -> d*q;
    Q4_0 {fp16 d; uint8 qs[16]} -> d*(nibble - 8), low nibbles elements 0..15, high nibbles
    16..31; F16 -> the half values;
  * activation rounding emulated in float32 exactly as ggml's quantize_row_q8_0 states it
    (d = amax/127, id = 1/d, q = round-half-away(x*id), d stored as fp16 round-to-nearest-
    even) and fp16 round-to-nearest-even for F16 weights;
  * everything else -- LayerNorm, attention, GELU-erf, the products and their sums -- in float64.

So the only differences left are the oracle's float32 rounding of terms and partial sums (about
5e-8 of the logit range) and the occasional activation that rounds to the other side of a
rounding step because its float64 input differed in the last bits. For Q8_0 / Q4_0 the step is
1/127 of the block's amax and such a flip is rare and small: every case stays within 1e-6 of the
logit range, against 4e-3 to 1e-2 for the planted mistakes. For F16 the step is an fp16 ulp,
flips are frequent enough to show in some seeds, and each one moves the logits by about 1e-5
to 2e-4 -- the same size as leaving the fp16 rounding out altogether. So F16 is judged over
twelve seeds: most agree within 1e-6 and none beyond a few flips, while the model without the
fp16 rounding misses every seed by more than 5e-5."""
import numpy as np
import pytest
from scipy.special import erf

from mgx import synth
from oracle import cpu_ref as R

T_F32, T_F16, T_Q4_0, T_Q8_0 = 0, 1, 2, 8
TOL = 1e-6


def dequant(ttype, ne0, ne1, data):
    """float64 [ne1][ne0] from ggml bytes."""
    raw = np.ascontiguousarray(data).view(np.uint8)
    if ttype == T_F32:
        return raw.view(np.float32).reshape(ne1, ne0).astype(np.float64)
    if ttype == T_F16:
        return raw.view(np.float16).reshape(ne1, ne0).astype(np.float64)
    nb = ne0 // 32
    if ttype == T_Q8_0:
        blk = raw.reshape(ne1, nb, 34)
        d = np.ascontiguousarray(blk[:, :, :2]).view(np.float16)[..., 0].astype(np.float64)
        q = np.ascontiguousarray(blk[:, :, 2:]).view(np.int8).astype(np.float64)
        return (q * d[..., None]).reshape(ne1, ne0)
    if ttype == T_Q4_0:
        blk = raw.reshape(ne1, nb, 18)
        d = np.ascontiguousarray(blk[:, :, :2]).view(np.float16)[..., 0].astype(np.float64)
        qs = blk[:, :, 2:].astype(np.int64)
        q = np.concatenate([(qs & 15) - 8, (qs >> 4) - 8], -1).astype(np.float64)
        return (q * d[..., None]).reshape(ne1, ne0)
    raise ValueError(ttype)


def act_q8(x, divisor=127.0):
    """ggml quantize_row_q8_0 of the float32 rounding of x, returned dequantized (float64)."""
    b = np.asarray(x, np.float64).astype(np.float32).reshape(*np.shape(x)[:-1], -1, 32)
    amax = np.abs(b).max(-1, keepdims=True)
    d = (amax / np.float32(divisor)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(d != 0, np.float32(1.0) / d, np.float32(0.0)).astype(np.float32)
    v = (b * inv).astype(np.float32).astype(np.float64)
    q = np.sign(v) * np.floor(np.abs(v) + 0.5)          # roundf: halves away from zero
    dh = d.astype(np.float16).astype(np.float64)          # the stored fp16 scale
    return (q * dh).reshape(np.shape(x))


def act_f16(x):
    return np.asarray(x, np.float64).astype(np.float32).astype(np.float16).astype(np.float64)


class Float64Model:
    """lm_forward / lm_layer (lm.h:152-259) in float64 over dequantized weights, with the
    activation rounding of each weight's type applied at every projection input."""

    def __init__(self, m, q8_divisor=127.0):
        self.c = m.config
        self.W, self.T = {}, {}
        for name, ttype, ne0, ne1, data in m.tensors:
            self.W[name] = dequant(ttype, ne0, ne1, data)
            self.T[name] = ttype
        self.div = q8_divisor

    def mm(self, x, name):
        t = self.T[name]
        if t in (T_Q8_0, T_Q4_0):
            x = act_q8(x, self.div)
        elif t == T_F16:
            x = act_f16(x)
        else:
            x = np.asarray(x, np.float64).astype(np.float32).astype(np.float64)
        return x @ self.W[name].T

    @staticmethod
    def ln(x, w, b, eps):
        mu = x.mean(-1, keepdims=True)
        var = ((x - mu) ** 2).mean(-1, keepdims=True)
        return (x - mu) / np.sqrt(var + eps) * w + b

    @staticmethod
    def attend(q, k, v, causal):
        s = np.einsum("thd,uhd->htu", q, k) / np.sqrt(q.shape[-1])
        if causal:
            T, U = q.shape[0], k.shape[0]
            s = np.where(np.arange(U)[None, :] <= (np.arange(T) + U - T)[:, None], s, -np.inf)
        p = np.exp(s - s.max(-1, keepdims=True))
        p /= p.sum(-1, keepdims=True)
        return np.einsum("htu,uhd->thd", p, v)

    def forward(self, ids, t5, n_seq, cross):
        """logits [n_seq][n_q][card] of the last of ids.shape[1] tokens fed from position 0."""
        c, W = self.c, self.W
        d, H, hd, T, eps = c.dim, c.heads, c.head_dim, ids.shape[1], c.norm_eps
        i = np.arange(d // 2)
        pos = np.arange(T)[:, None] / np.power(c.max_period, i / c.pos_denominator)
        pe = np.concatenate([np.cos(pos), np.sin(pos)], 1).astype(np.float32).astype(np.float64)
        emb = sum(W[f"lm.emb.{q}.weight"][ids[q]] for q in range(c.n_q))
        x = np.repeat((pe + emb)[None], n_seq, 0)
        if cross:
            ctx = self.mm(t5, "lm.cond_proj.weight") + W["lm.cond_proj.bias"][0]
        for l in range(c.layers):
            p = f"lm.{l}."
            nw = lambda k: (W[p + k + ".weight"][0], W[p + k + ".bias"][0])
            for n in range(n_seq):
                qkv = self.mm(self.ln(x[n], *nw("norm1"), eps), p + "self.qkv.weight")
                q, k, v = (qkv[:, j * d:(j + 1) * d].reshape(T, H, hd) for j in range(3))
                x[n] = x[n] + self.mm(self.attend(q, k, v, True).reshape(T, d), p + "self.out.weight")
                if cross and n == 0:   # the null stream's memory is zero: its block adds exactly 0
                    cq = self.mm(self.ln(x[n], *nw("norm_cross"), eps), p + "cross.q.weight").reshape(T, H, hd)
                    kv = self.mm(ctx, p + "cross.kv.weight")
                    ck, cv = kv[:, :d].reshape(-1, H, hd), kv[:, d:].reshape(-1, H, hd)
                    x[n] = x[n] + self.mm(self.attend(cq, ck, cv, False).reshape(T, d), p + "cross.out.weight")
                f = self.mm(self.ln(x[n], *nw("norm2"), eps), p + "ff.0.weight")
                f = (0.5 * f * (1 + erf(f / np.sqrt(2)))).astype(np.float32).astype(np.float64)
                x[n] = x[n] + self.mm(f, p + "ff.2.weight")
        xl = self.ln(x[:, -1], W["lm.out_norm.weight"][0], W["lm.out_norm.bias"][0], eps)
        return np.stack([np.stack([self.mm(xl[n], f"lm.head.{q}.weight") for q in range(c.n_q)])
                         for n in range(n_seq)])


SMALL = dict(dim=64, layers=2, heads=4, ff_dim=256, card=32, n_ctx=3)
CASES = [(shape, wtype, std) for shape in ("tiny", SMALL) for wtype in (T_Q8_0, T_Q4_0) for std in (0.02, 0.15)]


def rel_err(got, want):
    return float(np.abs(got - want).max() / (want.max() - want.min()))


def run_oracle(m, ids, t5, n_seq, tensors=None):
    rm = R.RefModel(m.config, tensors if tensors is not None else m.tensors)
    dec = R.RefDecoder(rm, 16, n_seq, t5, True)
    a = dec.forward(ids[:, :-1])
    b = dec.forward(ids[:, -1:])
    return a, b


@pytest.mark.parametrize("shape,wtype,std", CASES)
def test_quantized_forward_matches_float64(shape, wtype, std):
    m = synth.SyntheticModel(shape, wtype, seed=31, std=std)
    c = m.config
    t5 = synth.synth_memory(7, 5 if shape == "tiny" else 3)
    ids = synth.synth_codes(8, c.n_q, 10, c.card + 1)
    ref = Float64Model(m)
    pre, step = run_oracle(m, ids, t5, 2)
    want_pre = ref.forward(ids[:, :-1], t5, 2, True)
    want_step = ref.forward(ids, t5, 2, True)
    assert rel_err(pre, want_pre) <= TOL, rel_err(pre, want_pre)
    assert rel_err(step, want_step) <= TOL, rel_err(step, want_step)


def test_f16_forward_matches_float64_over_seeds():
    errs, unrounded = [], []
    for seed in range(12):
        m = synth.SyntheticModel(SMALL, T_F16, seed=seed)
        c = m.config
        t5 = synth.synth_memory(seed, 3)
        ids = synth.synth_codes(seed, c.n_q, 6, c.card + 1)
        _, got = run_oracle(m, ids, t5, 2)
        ref = Float64Model(m)
        errs.append(rel_err(got, ref.forward(ids, t5, 2, True)))
        ref.T = {k: (T_F32 if v == T_F16 else v) for k, v in ref.T.items()}
        unrounded.append(rel_err(got, ref.forward(ids, t5, 2, True)))
    assert sum(e <= TOL for e in errs) >= 8, errs
    assert max(errs) <= 5e-4, errs
    assert min(unrounded) > 5e-5, unrounded


def swap_nibbles(tensors):
    out = []
    for name, ttype, ne0, ne1, data in tensors:
        if ttype == T_Q4_0:
            blk = np.ascontiguousarray(data).view(np.uint8).reshape(-1, 18).copy()
            blk[:, 2:] = ((blk[:, 2:] & 15) << 4) | (blk[:, 2:] >> 4)
            data = blk.reshape(-1)
        out.append((name, ttype, ne0, ne1, data))
    return out


def test_planted_nibble_order_is_caught():
    """An oracle that read Q4_0 nibbles in the other order (high nibble = element j) is the
    oracle run on nibble-swapped bytes; the float64 model of the true bytes must reject it."""
    m = synth.SyntheticModel("tiny", T_Q4_0, seed=31, std=0.15)
    c = m.config
    t5 = synth.synth_memory(7, 5)
    ids = synth.synth_codes(8, c.n_q, 10, c.card + 1)
    want = Float64Model(m).forward(ids, t5, 2, True)
    _, good = run_oracle(m, ids, t5, 2)
    _, bad = run_oracle(m, ids, t5, 2, swap_nibbles(m.tensors))
    assert rel_err(good, want) <= TOL
    assert rel_err(bad, want) > 100 * TOL, rel_err(bad, want)


def test_planted_activation_scale_is_caught():
    """Activation blocks scaled by amax/128 instead of amax/127 (an off-by-one in ggml's
    quantize_row_q8_0) move the logits far beyond the tolerance: the test can see the
    activation quantizer, not only the weights."""
    m = synth.SyntheticModel("tiny", T_Q8_0, seed=31, std=0.15)
    c = m.config
    t5 = synth.synth_memory(7, 5)
    ids = synth.synth_codes(8, c.n_q, 10, c.card + 1)
    _, got = run_oracle(m, ids, t5, 2)
    assert rel_err(got, Float64Model(m).forward(ids, t5, 2, True)) <= TOL
    assert rel_err(got, Float64Model(m, q8_divisor=128.0).forward(ids, t5, 2, True)) > 100 * TOL


def test_unquantized_activations_are_caught():
    """The same comparison without the activation rounding (float64 activations against the
    quantized weights) is far outside the tolerance, so the rounding emulation is what agrees."""
    m = synth.SyntheticModel("tiny", T_Q8_0, seed=31, std=0.15)
    c = m.config
    t5 = synth.synth_memory(7, 5)
    ids = synth.synth_codes(8, c.n_q, 10, c.card + 1)
    _, got = run_oracle(m, ids, t5, 2)
    ref = Float64Model(m)
    ref.T = {k: T_F32 for k in ref.T}
    assert rel_err(got, ref.forward(ids, t5, 2, True)) > 100 * TOL


def test_block_decoders_on_known_bytes():
    """The numpy block decoders on hand-made blocks: Q8_0 d=0.5, q=-128..; Q4_0 nibbles."""
    q8 = np.zeros(34, np.uint8)
    q8[:2] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)
    q8[2:] = np.arange(-16, 16, dtype=np.int8).view(np.uint8)
    assert np.array_equal(dequant(T_Q8_0, 32, 1, q8)[0], 0.5 * np.arange(-16, 16))
    q4 = np.zeros(18, np.uint8)
    q4[:2] = np.frombuffer(np.float16(2.0).tobytes(), np.uint8)
    q4[2:] = (np.arange(16) | ((15 - np.arange(16)) << 4)).astype(np.uint8)
    want = 2.0 * (np.concatenate([np.arange(16), 15 - np.arange(16)]) - 8)
    assert np.array_equal(dequant(T_Q4_0, 32, 1, q4)[0], want)
    # the activation emulation: half away from zero, fp16 scale
    x = np.zeros(32)
    x[0], x[1], x[2] = 127.0, 0.5, -0.5
    got = act_q8(x)
    assert got[0] == 127.0 and got[1] == 1.0 and got[2] == -1.0
