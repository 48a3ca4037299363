"""Seeded synthetic MusicGen LMs in ggml tensor formats (libmgx_synth.so).

Every 2-D matrix is N(0, 0.02) -- embeddings [dim, card+1], heads, qkv, out, cross.q,
cross.kv, cross.out, ff.0, ff.2 and cond_proj [cond_dim, dim] -- and cond_proj.bias is
N(0, 0.02); LayerNorms are weight 1, bias 0. Matrices are stored as the requested ggml type
(F32 0, F16 1, Q4_0 2, Q8_0 8); vectors stay F32. Names follow the converter's GGUF contract
(tools/convert_musicgen_lm.py:149-210)."""
import ctypes as C
import os

import numpy as np

from .lib import LmConfig, T5Config

_HERE = os.path.dirname(os.path.abspath(__file__))
SYNTH_PATH = os.path.join(os.path.dirname(_HERE), "libmgx_synth.so")

# MusicGen LM shapes (hd 64, n_q 4, card 2048, T5-base memory width 768) plus a tiny one.
SHAPES = {
    "tiny": dict(dim=128, layers=2, heads=2, ff_dim=512, card=256, n_ctx=5),
    # one or two layers at the real widths: the GEMV shapes of the small / medium / large LMs
    "mini1024": dict(dim=1024, layers=2, heads=16, ff_dim=4096, card=256, n_ctx=6),
    "mini1536": dict(dim=1536, layers=1, heads=24, ff_dim=6144, card=256, n_ctx=7),
    "mini2048": dict(dim=2048, layers=1, heads=32, ff_dim=8192, card=256, n_ctx=9),
    "small": dict(dim=1024, layers=24, heads=16, ff_dim=4096, card=2048, n_ctx=12),
    "medium": dict(dim=1536, layers=48, heads=24, ff_dim=6144, card=2048, n_ctx=24),
    "large": dict(dim=2048, layers=48, heads=32, ff_dim=8192, card=2048, n_ctx=32),
}

_synth = None


def _lib():
    global _synth
    if _synth is None:
        if not os.path.exists(SYNTH_PATH):
            raise RuntimeError(f"{SYNTH_PATH} is not built; run __graft_entry__.build()")
        L = C.CDLL(SYNTH_PATH)
        L.mgx_synth_seed.restype = C.c_uint64
        L.mgx_synth_seed.argtypes = [C.c_uint64, C.c_char_p]
        L.mgx_synth_normal.argtypes = [C.c_uint64, C.c_float, C.c_void_p, C.c_uint64]
        L.mgx_synth_codes.argtypes = [C.c_uint64, C.c_int32, C.c_void_p, C.c_uint64]
        L.mgx_row_bytes.restype = C.c_uint64
        L.mgx_row_bytes.argtypes = [C.c_int, C.c_int64]
        L.mgx_synth_tensor.argtypes = [C.c_uint64, C.c_int, C.c_int64, C.c_int64, C.c_float, C.c_float, C.c_void_p]
        L.mgx_pack.argtypes = [C.c_int, C.c_void_p, C.c_int64, C.c_int64, C.c_void_p]
        _synth = L
    return _synth


def make_config(shape, cfg_coef=3.0, **over):
    s = dict(SHAPES[shape]) if isinstance(shape, str) else dict(shape)
    s.update(over)
    c = LmConfig()
    c.dim, c.layers, c.heads = s["dim"], s["layers"], s["heads"]
    c.head_dim = s["dim"] // s["heads"]
    c.ff_dim = s["ff_dim"]
    c.cond_dim = s.get("cond_dim", 768)
    c.n_q = s.get("n_q", 4)
    c.card = s["card"]
    c.special_token_id = s["card"]
    c.pos_denominator = s.get("pos_denominator", s["dim"] // 2 - 1)
    c.max_period, c.norm_eps, c.cfg_coef = 10000.0, 1e-5, cfg_coef
    return c


def synth_memory(seed, n_ctx, cond_dim=768):
    """The T5-base stand-in: [n_ctx][cond_dim] f32 N(0, 1)."""
    out = np.empty((n_ctx, cond_dim), np.float32)
    _lib().mgx_synth_normal(_lib().mgx_synth_seed(seed, b"t5.memory"), 1.0, out.ctypes.data, out.size)
    return out


def synth_codes(seed, n_q, length, card=2048):
    """Uniform prompt codes [n_q][length] in [0, card)."""
    out = np.empty((n_q, length), np.int32)
    _lib().mgx_synth_codes(_lib().mgx_synth_seed(seed, b"prompt.codes"), card, out.ctypes.data, out.size)
    return out


# The projections an adapter may target (lora.h:201-202) and their (in, out) widths.
def adapter_shapes(config):
    d, f = config.dim, config.ff_dim
    return {"self.qkv": (d, 3 * d), "self.out": (d, d), "cross.q": (d, d), "cross.kv": (d, 2 * d),
            "cross.out": (d, d), "ff.0": (d, f), "ff.2": (f, d)}


def synth_adapters(config, rank=16, targets=("self.qkv", "ff.0", "ff.2"), dora=True, alpha=None, strength=1.0,
                   seed=0):
    """Rank-`rank` adapters on `targets` of every layer, as dicts for Model.set_adapters:
    A [rank][in] and B [out][rank] N(0, 0.01); for DoRA rows a magnitude [out] U(0.9, 1.1).
    alpha defaults to rank (scale 1). Streams are seeded per tensor name, as the weights are
    (stem + ".lora_A" / ".lora_B" / ".magnitude", the adapter GGUF names of lora.h:125-150)."""
    lib = _lib()
    widths = adapter_shapes(config)
    out = []
    for l in range(config.layers):
        for t in targets:
            i, o = widths[t]
            stem = f"lm.{l}.{t}.weight"
            A = np.empty((rank, i), np.float32)
            B = np.empty((o, rank), np.float32)
            lib.mgx_synth_normal(lib.mgx_synth_seed(seed, (stem + ".lora_A").encode()), 0.01, A.ctypes.data, A.size)
            lib.mgx_synth_normal(lib.mgx_synth_seed(seed, (stem + ".lora_B").encode()), 0.01, B.ctypes.data, B.size)
            a = dict(target=stem, rank=rank, alpha=float(rank if alpha is None else alpha), strength=float(strength),
                     A=A, B=B, magnitude=None)
            if dora:
                u = np.empty(o, np.int32)
                lib.mgx_synth_codes(lib.mgx_synth_seed(seed, (stem + ".magnitude").encode()), 1 << 24, u.ctypes.data, o)
                a["magnitude"] = (0.9 + 0.2 * ((u.astype(np.float64) + 0.5) / float(1 << 24))).astype(np.float32)
            out.append(a)
    return out


def pack(ttype, x):
    """Packs a float32 [rows][ne0] array into ggml bytes of `ttype`."""
    x = np.ascontiguousarray(x, np.float32)
    rows, ne0 = x.shape
    out = np.empty(int(_lib().mgx_row_bytes(ttype, ne0)) * rows, np.uint8)
    if _lib().mgx_pack(ttype, x.ctypes.data, ne0, rows, out.ctypes.data):
        raise ValueError("cannot pack this shape")
    return out


class SyntheticModel:
    """Tensors of one synthetic LM: list of (name, type, ne0, ne1, uint8 bytes)."""

    def __init__(self, shape, wtype, seed=0, std=0.02, cfg_coef=3.0, **over):
        self.config = make_config(shape, cfg_coef, **over)
        self.wtype = wtype
        self.seed = seed
        c = self.config
        L = _lib()
        self.tensors = []

        def mat(name, ne0, ne1, ttype=wtype, sd=std, const=0.0):
            buf = np.empty(int(L.mgx_row_bytes(ttype, ne0)) * ne1, np.uint8)
            if L.mgx_synth_tensor(L.mgx_synth_seed(seed, name.encode()), ttype, ne0, ne1, sd, const,
                                  buf.ctypes.data):
                raise ValueError(f"cannot synthesize {name}")
            self.tensors.append((name, ttype, ne0, ne1, buf))

        def vec(name, n, sd=0.0, const=0.0):
            mat(name, n, 1, 0, sd, const)

        d, F = c.dim, c.ff_dim
        for q in range(c.n_q):
            mat(f"lm.emb.{q}.weight", d, c.card + 1)
        mat("lm.cond_proj.weight", c.cond_dim, d)
        vec("lm.cond_proj.bias", d, sd=std)
        for i in range(c.layers):
            p = f"lm.{i}."
            for norm in ("norm1", "norm_cross", "norm2"):
                vec(p + norm + ".weight", d, const=1.0)
                vec(p + norm + ".bias", d, const=0.0)
            mat(p + "self.qkv.weight", d, 3 * d)
            mat(p + "self.out.weight", d, d)
            mat(p + "cross.q.weight", d, d)
            mat(p + "cross.kv.weight", d, 2 * d)
            mat(p + "cross.out.weight", d, d)
            mat(p + "ff.0.weight", d, F)
            mat(p + "ff.2.weight", F, d)
        vec("lm.out_norm.weight", d, const=1.0)
        vec("lm.out_norm.bias", d, const=0.0)
        for q in range(c.n_q):
            mat(f"lm.head.{q}.weight", d, c.card)

    def tensor(self, name):
        for t in self.tensors:
            if t[0] == name:
                return t
        raise KeyError(name)

    def replace(self, name, ttype, values):
        """Swaps one tensor for caller values (float32 [ne1][ne0]) packed as `ttype`."""
        for i, t in enumerate(self.tensors):
            if t[0] == name:
                v = np.ascontiguousarray(values, np.float32)
                self.tensors[i] = (name, ttype, v.shape[1], v.shape[0], pack(ttype, v) if ttype != 0 else
                                   v.view(np.uint8).reshape(-1).copy())
                return
        raise KeyError(name)

    def nbytes(self):
        return sum(t[4].nbytes for t in self.tensors)


# T5 encoder shapes: T5-base (t5.h:20-29) and small ones for tests.
T5_SHAPES = {
    "t5-tiny": dict(dim=128, layers=2, heads=2, intermediate=256, vocab=300),
    "t5-mini": dict(dim=768, layers=1, heads=12, intermediate=3072, vocab=1000),
    "t5-base": dict(dim=768, layers=12, heads=12, intermediate=3072, vocab=32128),
}


def make_t5_config(shape, **over):
    s = dict(T5_SHAPES[shape]) if isinstance(shape, str) else dict(shape)
    s.update(over)
    c = T5Config()
    c.dim, c.layers, c.heads, c.head_dim = s["dim"], s["layers"], s["heads"], s.get("head_dim", 64)
    c.intermediate, c.vocab = s["intermediate"], s["vocab"]
    c.relative_buckets, c.relative_max_distance = s.get("relative_buckets", 32), s.get("relative_max_distance", 128)
    c.eps = s.get("eps", 1e-6)
    return c


class SyntheticT5:
    """Tensors of one synthetic T5 encoder (names of tools/convert_t5.py:107-119): embedding
    N(0, 1) and linears N(0, 0.04) (wi, wo N(0, 0.03)) in the requested ggml type, the relative
    bias table [buckets][heads] N(0, 1) and RMS norm weights 1 + N(0, 0.1), f32."""

    def __init__(self, shape, wtype, seed=0, **over):
        self.config = c = make_t5_config(shape, **over)
        self.wtype = wtype
        L = _lib()
        self.tensors = []

        def mat(name, ne0, ne1, sd, ttype=wtype):
            buf = np.empty(int(L.mgx_row_bytes(ttype, ne0)) * ne1, np.uint8)
            if L.mgx_synth_tensor(L.mgx_synth_seed(seed, name.encode()), ttype, ne0, ne1, sd, 0.0, buf.ctypes.data):
                raise ValueError(f"cannot synthesize {name}")
            self.tensors.append((name, ttype, ne0, ne1, buf))

        def norm(name, n):
            v = np.empty(n, np.float32)
            L.mgx_synth_normal(L.mgx_synth_seed(seed, name.encode()), 0.1, v.ctypes.data, n)
            self.tensors.append((name, 0, n, 1, (v + np.float32(1.0)).view(np.uint8).copy()))

        d, inner, F = c.dim, c.heads * c.head_dim, c.intermediate
        mat("te.embed.weight", d, c.vocab, 1.0)
        mat("te.relative_attention_bias.weight", c.heads, c.relative_buckets, 1.0, ttype=0)
        for i in range(c.layers):
            p = f"te.{i}."
            norm(p + "attn_norm.weight", d)
            for w in ("q", "k", "v"):
                mat(p + w + ".weight", d, inner, 0.04)
            mat(p + "o.weight", inner, d, 0.04)
            norm(p + "ffn_norm.weight", d)
            mat(p + "wi.weight", d, F, 0.03)
            mat(p + "wo.weight", F, d, 0.03)
        norm("te.norm.weight", d)


def synth_ids(seed, n, vocab):
    """Token ids [n] uniform in [0, vocab)."""
    out = np.empty(n, np.int32)
    _lib().mgx_synth_codes(_lib().mgx_synth_seed(seed, b"t5.ids"), vocab, out.ctypes.data, n)
    return out


# SEANet codec shapes (SeanetConfig, src/ac/seanet.h:32-58): MusicGen's EnCodec 32 kHz and a
# tiny one whose odd ratio exercises the asymmetric transposed-conv trim.
CODEC_SHAPES = {
    "codec-tiny": dict(n_filters=4, ratios=[2, 3], latent_dim=8, rvq_n_q=2, rvq_bins=16, sample_rate=6000),
    "codec-mini": dict(n_filters=16, ratios=[4, 5], latent_dim=32, rvq_n_q=4, rvq_bins=64, sample_rate=32000),
    "encodec-32k": dict(n_filters=64, ratios=[8, 5, 4, 4], latent_dim=128, rvq_n_q=4, rvq_bins=2048,
                        sample_rate=32000),
}


def make_codec_config(shape, **over):
    s = dict(quantizer="rvq", activation="ELU", channels=1, n_residual_layers=1, kernel_size=7,
             residual_kernel_size=3, last_kernel_size=7, dilation_base=2, compress=2, lstm_layers=2)
    s.update(CODEC_SHAPES[shape] if isinstance(shape, str) else shape)
    s.update(over)
    hop = 1
    for r in s["ratios"]:
        hop *= r
    s["hop_length"] = hop
    s["frame_rate"] = s["sample_rate"] // hop
    s["encoder_dim"] = s["latent_dim"]
    return s


class SyntheticCodec:
    """The decoder half of a SEANet / EnCodec checkpoint as tools/convert_seanet.py names it
    (weight norm already fused): conv weights N(0, 1/sqrt(in * k)), biases N(0, 0.1), LSTM
    matrices U(-1/sqrt(H), 1/sqrt(H)), codebooks N(0, 1), all f32. `weights` maps names to
    numpy arrays in row-major ggml order (conv [out][in][k], transposed conv [out*k][in]);
    `tensors` lists (name, type, ne list, bytes) for the library."""

    def __init__(self, shape, seed=0, **over):
        self.config = c = make_codec_config(shape, **over)
        rng = np.random.default_rng(seed)
        W = {}

        def conv(name, cin, cout, k):
            W[name + ".weight"] = rng.normal(0, 1 / np.sqrt(cin * k), (cout, cin, k)).astype(np.float32)
            W[name + ".bias"] = rng.normal(0, 0.1, cout).astype(np.float32)

        bott = c["n_filters"] * 2 ** len(c["ratios"])
        conv("codec.decoder.in", c["latent_dim"], bott, c["kernel_size"])
        for l in range(c["lstm_layers"]):
            a = 1 / np.sqrt(bott)
            for m in ("w_ih", "w_hh"):
                W[f"codec.decoder.lstm.{l}.{m}"] = rng.uniform(-a, a, (4 * bott, bott)).astype(np.float32)
            W[f"codec.decoder.lstm.{l}.bias"] = rng.uniform(-2 * a, 2 * a, 4 * bott).astype(np.float32)
        mult = 2 ** len(c["ratios"])
        for s, ratio in enumerate(c["ratios"]):
            cin = c["n_filters"] * mult
            cout = cin // 2
            k = 2 * ratio
            p = f"codec.decoder.stage.{s}."
            W[p + "up.weight_col2im"] = rng.normal(0, 1 / np.sqrt(cin * 2), (cout * k, cin)).astype(np.float32)
            W[p + "up.bias"] = rng.normal(0, 0.1, cout).astype(np.float32)
            for j in range(c["n_residual_layers"]):
                hid = cout // c["compress"]
                conv(p + f"res.{j}.conv1", cout, hid, c["residual_kernel_size"])
                conv(p + f"res.{j}.conv2", hid, cout, 1)
            mult //= 2
        conv("codec.decoder.out", c["n_filters"], c["channels"], c["last_kernel_size"])
        for i in range(c["rvq_n_q"]):
            W[f"codec.rvq.{i}.embed"] = rng.normal(0, 1, (c["rvq_bins"], c["latent_dim"])).astype(np.float32)
        self.weights = W
        self.tensors = [(n, 0, list(a.shape[::-1]), a.view(np.uint8).reshape(-1)) for n, a in W.items()]

    def codes(self, seed, frames):
        rng = np.random.default_rng(seed)
        return rng.integers(0, self.config["rvq_bins"], (self.config["rvq_n_q"], frames)).astype(np.int32)
