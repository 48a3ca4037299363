"""ctypes binding of the oracle (oracle/libcpu_ref.so, built from oracle/cpu_ref.c).

TEST INFRASTRUCTURE: the CPU restatement of the reference's MusicGen LM decode path, used
only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the checker and the
timed CPU baseline. The product never imports this module.

Also binds oracle/_ref/libref_host.so -- the reference's own header-only sampling, RNG and
delay-pattern code (src/mg/sampling.h, src/rng.h, src/mg/pattern.h) compiled from its
sources -- when it has been built (it needs the reference tree, so it may be absent)."""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libcpu_ref.so")
REF_HOST_PATH = os.path.join(HERE, "_ref", "libref_host.so")


class RefConfig(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("dim", "layers", "heads", "head_dim", "ff_dim", "cond_dim", "n_q",
                                         "card", "special_token_id", "pos_denominator")] + \
               [(n, C.c_float) for n in ("max_period", "norm_eps", "cfg_coef")]


class RefT5Config(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("dim", "layers", "heads", "head_dim", "intermediate", "vocab",
                                         "relative_buckets", "relative_max_distance")] + [("eps", C.c_float)]


class RefTensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("type", C.c_int32), ("ne0", C.c_int64), ("ne1", C.c_int64),
                ("data", C.c_void_p)]


class RefAdapter(C.Structure):
    _fields_ = [("target", C.c_char_p), ("A", C.c_void_p), ("B", C.c_void_p), ("magnitude", C.c_void_p),
                ("rank", C.c_int32), ("alpha", C.c_float), ("strength", C.c_float)]


class RefGenParams(C.Structure):
    _fields_ = [("max_gen_len", C.c_int32), ("use_sampling", C.c_int32), ("temperature", C.c_float),
                ("top_k", C.c_int32), ("cfg_coef", C.c_float), ("seed", C.c_uint64)]


class RefReport(C.Structure):
    _fields_ = [("cache_bytes", C.c_size_t), ("prefill_tokens", C.c_int32), ("decode_steps", C.c_int32),
                ("forwards", C.c_int32), ("prefill_seconds", C.c_double), ("decode_seconds", C.c_double)]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built (make -C oracle)")
        L = C.CDLL(LIB_PATH)
        P = C.c_void_p
        L.ref_last_error.restype = C.c_char_p
        L.ref_fp16_to_fp32.restype = C.c_float
        L.ref_fp16_to_fp32.argtypes = [C.c_uint16]
        L.ref_fp32_to_fp16.restype = C.c_uint16
        L.ref_fp32_to_fp16.argtypes = [C.c_float]
        for f in ("ref_exp", "ref_erf"):
            getattr(L, f).restype = C.c_double
            getattr(L, f).argtypes = [C.c_double]
        for f in ("ref_expf", "ref_erff", "ref_gelu_erf"):
            getattr(L, f).restype = C.c_float
            getattr(L, f).argtypes = [C.c_float]
        L.ref_quantize_q8_0.argtypes = [P, C.c_int, P]
        L.ref_layer_norm.argtypes = [P, C.c_int, P, P, C.c_float, P]
        L.ref_sin_positions.argtypes = [C.c_int, C.c_int, C.c_int, C.c_int, C.c_float, P]
        L.ref_attend.argtypes = [P, C.c_int, C.c_int, P, P, C.c_int, P, C.c_float, P]
        L.ref_model_create.restype = P
        L.ref_model_create.argtypes = [C.POINTER(RefConfig), C.POINTER(RefTensor), C.c_int, C.POINTER(RefAdapter),
                                       C.c_int]
        L.ref_model_destroy.argtypes = [P]
        L.ref_decoder_create.restype = P
        L.ref_decoder_create.argtypes = [P, C.c_int, C.c_int, P, C.c_int, C.c_int, C.c_int]
        L.ref_decoder_destroy.argtypes = [P]
        L.ref_decoder_used.argtypes = [P]
        L.ref_decoder_cache_bytes.restype = C.c_size_t
        L.ref_decoder_cache_bytes.argtypes = [P]
        L.ref_forward.argtypes = [P, P, C.c_int, P]
        L.ref_rng_size.restype = C.c_size_t
        L.ref_rng_seed.argtypes = [P, C.c_uint64]
        L.ref_rng_next.restype = C.c_uint32
        L.ref_rng_next.argtypes = [P]
        L.ref_rng_uniform.restype = C.c_float
        L.ref_rng_uniform.argtypes = [P]
        L.ref_argmax.argtypes = [P, C.c_int]
        L.ref_softmax_into.argtypes = [P, C.c_int, C.c_float, P]
        L.ref_softmax_into_devexp.argtypes = [P, C.c_int, C.c_float, P]
        L.ref_softmax_exp_compare.argtypes = [P, C.c_int, C.c_int, C.c_float, C.POINTER(C.c_longlong),
                                              C.POINTER(C.c_longlong)]
        L.ref_top_k_filter.argtypes = [P, C.c_int, C.c_int]
        L.ref_categorical.argtypes = [P, C.c_int, C.c_double, P]
        L.ref_sample_top_k.argtypes = [P, C.c_int, C.c_int, C.c_float, P, P]
        L.ref_pattern_steps.argtypes = [C.c_int, C.c_int]
        L.ref_build_pattern.argtypes = [C.c_int, C.c_int, P, C.c_int32, P]
        L.ref_revert_pattern.argtypes = [C.c_int, C.c_int, P, C.c_int32, P]
        L.ref_pattern_mask.argtypes = [C.c_int, C.c_int, P]
        L.ref_use_guidance.argtypes = [C.c_float, C.c_int]
        L.ref_generate.argtypes = [P, P, C.c_int, C.c_int, P, C.c_int, C.POINTER(RefGenParams), C.c_int, C.c_int, P, P,
                                   P, C.POINTER(RefReport)]
        L.ref_set_threads.argtypes = [C.c_int]
        L.ref_t5_bucket.argtypes = [C.c_int, C.c_int, C.c_int]
        L.ref_rms_norm.argtypes = [P, C.c_int, P, C.c_float, P]
        L.ref_t5_encode.argtypes = [C.POINTER(RefT5Config), C.POINTER(RefTensor), C.c_int, P, C.c_int, P]
        L.ref_convention.restype = C.c_int
        _lib = L
    return _lib


_ref_host = None


def ref_host():
    """The reference's own sampling / RNG / pattern code, or None when not built here."""
    global _ref_host
    if _ref_host is None:
        if not os.path.exists(REF_HOST_PATH):
            return None
        L = C.CDLL(REF_HOST_PATH)
        P = C.c_void_p
        L.refx_argmax.argtypes = [P, C.c_int]
        L.refx_softmax_into.argtypes = [P, C.c_int, C.c_float, P]
        L.refx_top_k_filter.argtypes = [P, C.c_int, C.c_int]
        L.refx_sample_top_k_seq.argtypes = [P, C.c_int, C.c_int, C.c_float, C.c_ulonglong, C.c_int, P]
        L.refx_sample_rows.argtypes = [P, C.c_int, C.c_int, C.c_int, C.c_float, C.c_ulonglong, P]
        L.refx_rng_uniforms.argtypes = [C.c_ulonglong, C.c_int, P]
        L.refx_rng_raw.argtypes = [C.c_ulonglong, C.c_int, P]
        L.refx_pattern_steps.argtypes = [C.c_int, C.c_int]
        L.refx_build_pattern.argtypes = [C.c_int, C.c_int, P, C.c_int, P]
        L.refx_revert_pattern.argtypes = [C.c_int, C.c_int, P, C.c_int, P]
        L.refx_pattern_mask.argtypes = [C.c_int, C.c_int, P]
        L.refx_first_step_with_timestep.argtypes = [C.c_int, C.c_int, C.c_int]
        _ref_host = L
    return _ref_host


def ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def err():
    return lib().ref_last_error().decode()


def set_threads(n):
    lib().ref_set_threads(int(n))


def config_from(c):
    r = RefConfig()
    for name, _ in RefConfig._fields_:
        setattr(r, name, getattr(c, name))
    return r


class RefModel:
    """The oracle's view of a model: the same ggml tensor bytes the HIP library uploads."""

    def __init__(self, config, tensors, adapters=None):
        self.config = config
        self._keep = []
        arr = (RefTensor * len(tensors))()
        for i, (name, ttype, ne0, ne1, data) in enumerate(tensors):
            b = name.encode()
            self._keep.append(b)
            arr[i].name, arr[i].type, arr[i].ne0, arr[i].ne1, arr[i].data = b, ttype, ne0, ne1, data.ctypes.data
        ads = None
        nad = 0
        if adapters:
            nad = len(adapters)
            ads = (RefAdapter * nad)()
            for i, a in enumerate(adapters):
                b = a["target"].encode()
                self._keep += [b, a["A"], a["B"], a.get("magnitude")]
                ads[i].target = b
                ads[i].A = a["A"].ctypes.data
                ads[i].B = a["B"].ctypes.data
                ads[i].magnitude = a["magnitude"].ctypes.data if a.get("magnitude") is not None else None
                ads[i].rank, ads[i].alpha, ads[i].strength = a["rank"], a["alpha"], a.get("strength", 1.0)
        self.cfg = config_from(config)
        self.handle = lib().ref_model_create(C.byref(self.cfg), arr, len(tensors), ads, nad)
        if not self.handle:
            raise RuntimeError(err())
        self._tensors = tensors

    def __del__(self):
        try:
            if self.handle:
                lib().ref_model_destroy(self.handle)
        except Exception:
            pass

    def generate(self, t5_hidden, prompt_codes, prompt_len, max_gen_len, use_sampling=True, temperature=1.0,
                 top_k=250, cfg_coef=3.0, seed=0, description_empty=False, recompute_cross_kv=False,
                 max_forwards=0, step_logits=False):
        c = self.config
        p = RefGenParams(max_gen_len, 1 if use_sampling else 0, temperature, top_k, cfg_coef, seed)
        T = max_gen_len
        S = T + c.n_q
        start = prompt_len + 1
        codes = np.zeros((c.n_q, T), np.int32)
        first = np.zeros((c.n_q, c.card), np.float32)
        steps = np.zeros((S - start, c.n_q, c.card), np.float32) if step_logits else None
        rep = RefReport()
        t5 = np.ascontiguousarray(t5_hidden, np.float32)
        prompt = np.ascontiguousarray(prompt_codes, np.int32) if prompt_len else None
        rc = lib().ref_generate(self.handle, ptr(t5), t5.shape[0], 1 if description_empty else 0, ptr(prompt),
                                prompt_len, C.byref(p), 1 if recompute_cross_kv else 0, max_forwards, ptr(codes),
                                ptr(first), ptr(steps), C.byref(rep))
        if rc:
            raise RuntimeError(err())
        return codes, first, rep, steps


class RefDecoder:
    """The oracle's Decoder (pipeline.cpp:36-195)."""

    def __init__(self, model, capacity, n_seq, t5_hidden=None, cross_attention=True, recompute_cross_kv=False):
        self.model = model
        self.n_seq = n_seq
        t5 = None if t5_hidden is None else np.ascontiguousarray(t5_hidden, np.float32)
        self._t5 = t5
        self.handle = lib().ref_decoder_create(model.handle, capacity, n_seq, ptr(t5), 0 if t5 is None else t5.shape[0],
                                               1 if cross_attention else 0, 1 if recompute_cross_kv else 0)
        if not self.handle:
            raise RuntimeError(err())

    def forward(self, ids):
        c = self.model.config
        ids = np.ascontiguousarray(ids, np.int32)
        out = np.zeros((self.n_seq, c.n_q, c.card), np.float32)
        if lib().ref_forward(self.handle, ptr(ids), ids.shape[1], ptr(out)):
            raise RuntimeError(err())
        return out

    def used(self):
        return lib().ref_decoder_used(self.handle)

    def cache_bytes(self):
        return lib().ref_decoder_cache_bytes(self.handle)

    def __del__(self):
        try:
            if self.handle:
                lib().ref_decoder_destroy(self.handle)
        except Exception:
            pass


class RefRng:
    def __init__(self, seed):
        self.buf = C.create_string_buffer(int(lib().ref_rng_size()))
        lib().ref_rng_seed(self.buf, seed)

    def next(self):
        return lib().ref_rng_next(self.buf)

    def uniform(self):
        return lib().ref_rng_uniform(self.buf)


def t5_bucket(relative_position, num_buckets=32, max_distance=128):
    return lib().ref_t5_bucket(int(relative_position), num_buckets, max_distance)


def rms_norm(x, w, eps):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    y = np.empty_like(x)
    lib().ref_rms_norm(ptr(x), x.size, ptr(w), eps, ptr(y))
    return y


def t5_encode(config, tensors, ids):
    """The oracle's T5 encoder: last_hidden_state [seq][dim] of ids [seq] (t5.h:85-140)."""
    cfg = RefT5Config()
    for name, _ in RefT5Config._fields_:
        setattr(cfg, name, getattr(config, name))
    keep = []
    arr = (RefTensor * len(tensors))()
    for i, (name, ttype, ne0, ne1, data) in enumerate(tensors):
        b = name.encode()
        keep.append(b)
        arr[i].name, arr[i].type, arr[i].ne0, arr[i].ne1, arr[i].data = b, ttype, ne0, ne1, data.ctypes.data
    ids = np.ascontiguousarray(ids, np.int32)
    out = np.zeros((ids.size, config.dim), np.float32)
    if lib().ref_t5_encode(C.byref(cfg), arr, len(tensors), ptr(ids), ids.size, ptr(out)):
        raise RuntimeError(err())
    return out
