"""ctypes bindings over include/mgx.h (libmgx.so, built in place by the package Makefile).

Loading fails loudly when the library is missing: there is no host fallback."""
import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_PKG = os.path.dirname(_HERE)
LIB_PATH = os.path.join(_PKG, "libmgx.so")


class MgxError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"mgx error {code}: {msg}")
        self.code = code


class LmConfig(C.Structure):
    """mgx_lm_config = ac::LmConfig (src/mg/lm.h:42-93)."""
    _fields_ = [(n, C.c_int32) for n in ("dim", "layers", "heads", "head_dim", "ff_dim", "cond_dim", "n_q",
                                         "card", "special_token_id", "pos_denominator")] + \
               [(n, C.c_float) for n in ("max_period", "norm_eps", "cfg_coef")]


class T5Config(C.Structure):
    """mgx_t5_config = ac::T5EncoderConfig (src/ac/t5.h:20-44)."""
    _fields_ = [(n, C.c_int32) for n in ("dim", "layers", "heads", "head_dim", "intermediate", "vocab",
                                         "relative_buckets", "relative_max_distance")] + [("eps", C.c_float)]


class CodecConfig(C.Structure):
    """mgx_codec_config = ac::SeanetConfig (src/ac/seanet.h:32-92)."""
    _fields_ = [(n, C.c_int32) for n in ("channels", "n_filters", "n_residual_layers", "kernel_size",
                                         "residual_kernel_size", "last_kernel_size", "dilation_base", "compress",
                                         "lstm_layers", "latent_dim", "sample_rate", "hop_length", "frame_rate",
                                         "rvq", "rvq_n_q", "rvq_bins", "elu", "n_ratios")] + \
               [("ratios", C.c_int32 * 8)]

    @classmethod
    def of(cls, d):
        """From a SeanetConfig-like dict (mgx.synth.make_codec_config)."""
        c = cls()
        for n, _ in cls._fields_:
            if n in d and n != "ratios":
                setattr(c, n, int(d[n]))
        c.rvq = 1 if d.get("quantizer", "rvq") == "rvq" else 0
        c.elu = 1 if d.get("activation", "ELU") == "ELU" else 0
        c.n_ratios = len(d["ratios"])
        for i, r in enumerate(d["ratios"]):
            c.ratios[i] = r
        return c


class Tensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("type", C.c_int32), ("ne", C.c_int64 * 4), ("data", C.c_void_p),
                ("nbytes", C.c_uint64)]


class Adapter(C.Structure):
    _fields_ = [("target", C.c_char_p), ("A", C.c_void_p), ("B", C.c_void_p), ("magnitude", C.c_void_p),
                ("rank", C.c_int32), ("alpha", C.c_float), ("strength", C.c_float)]


class GenerateParams(C.Structure):
    """mgx_generate_params = ac::GenerateParams (src/mg/pipeline.h:25-34)."""
    _fields_ = [("max_gen_len", C.c_int32), ("use_sampling", C.c_int32), ("temperature", C.c_float),
                ("top_k", C.c_int32), ("cfg_coef", C.c_float), ("seed", C.c_uint64)]


class BatchRequest(C.Structure):
    """mgx_batch_request: one request of a lockstep batch."""
    _fields_ = [("t5_hidden", C.c_void_p), ("description_empty", C.c_int32), ("prompt_codes", C.c_void_p),
                ("params", GenerateParams)]


class ServerConfig(C.Structure):
    """mgx_server_config."""
    _fields_ = [("slots", C.c_int32), ("guided", C.c_int32), ("max_gen_len", C.c_int32), ("max_ctx", C.c_int32),
                ("keep_step_logits", C.c_int32), ("steps_per_round", C.c_int32)]


class ServerCounters(C.Structure):
    _fields_ = [("steps", C.c_int64), ("slot_steps", C.c_int64), ("served", C.c_int64), ("active", C.c_int32),
                ("queued", C.c_int32)]


PROGRESS_FN = C.CFUNCTYPE(None, C.c_void_p, C.c_int32, C.c_int32)


class GenerateReport(C.Structure):
    _fields_ = [("cache_bytes", C.c_uint64), ("prefill_tokens", C.c_int32), ("decode_steps", C.c_int32),
                ("forwards", C.c_int32), ("prefill_seconds", C.c_double), ("decode_seconds", C.c_double)]


EXPORTS = ["mgx_model_create", "mgx_model_set_adapters", "mgx_model_destroy", "mgx_stream_create", "mgx_forward",
           "mgx_stream_reset", "mgx_stream_used", "mgx_stream_forwards", "mgx_stream_cache_bytes",
           "mgx_stream_destroy", "mgx_use_guidance", "mgx_generate", "mgx_session_create", "mgx_session_step",
           "mgx_session_remaining", "mgx_session_finish", "mgx_session_destroy", "mgx_session_profile",
           "mgx_session_profile_read", "mgx_session_hip_stream", "mgx_batch_create", "mgx_batch_finish",
           "mgx_session_requests", "mgx_gguf_open", "mgx_gguf_close", "mgx_gguf_tensor_count", "mgx_gguf_tensor",
           "mgx_gguf_find_tensor", "mgx_gguf_u32", "mgx_gguf_f32", "mgx_gguf_string", "mgx_gguf_lm_config",
           "mgx_model_create_from_gguf", "mgx_model_set_adapters_from_gguf", "mgx_server_create",
           "mgx_server_generate", "mgx_server_stats", "mgx_server_destroy", "mgx_t5_create", "mgx_gguf_t5_config",
           "mgx_t5_create_from_gguf", "mgx_t5_encode", "mgx_t5_encode_static", "mgx_t5_destroy", "mgx_t5_relative_bucket", "mgx_codec_create",
           "mgx_gguf_codec_config", "mgx_codec_create_from_gguf", "mgx_codec_decode", "mgx_codec_decode_latent",
           "mgx_codec_destroy", "mgx_last_error"]

_lib = None


def load(path=None):
    """The loaded libmgx.so (raises if it has not been built)."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = path or LIB_PATH
    if not os.path.exists(p):
        raise MgxError(-2, f"{p} is not built; run __graft_entry__.build()")
    lib = C.CDLL(p)
    P = C.c_void_p
    lib.mgx_last_error.restype = C.c_char_p
    lib.mgx_model_create.argtypes = [C.POINTER(LmConfig), C.POINTER(Tensor), C.c_int32, C.POINTER(P)]
    lib.mgx_model_set_adapters.argtypes = [P, C.POINTER(Adapter), C.c_int32]
    lib.mgx_model_destroy.argtypes = [P]
    lib.mgx_model_destroy.restype = None
    lib.mgx_stream_create.argtypes = [P, C.c_int32, C.c_int32, P, C.c_int32, C.c_int32, C.POINTER(P)]
    lib.mgx_forward.argtypes = [P, P, C.c_int32, P]
    lib.mgx_stream_reset.argtypes = [P]
    lib.mgx_stream_used.argtypes = [P]
    lib.mgx_stream_forwards.argtypes = [P]
    lib.mgx_stream_cache_bytes.argtypes = [P]
    lib.mgx_stream_cache_bytes.restype = C.c_uint64
    lib.mgx_stream_destroy.argtypes = [P]
    lib.mgx_stream_destroy.restype = None
    lib.mgx_use_guidance.argtypes = [C.c_float, C.c_int32]
    lib.mgx_generate.argtypes = [P, P, C.c_int32, C.c_int32, P, C.c_int32, C.POINTER(GenerateParams), P, P, P,
                                 C.POINTER(GenerateReport)]
    lib.mgx_session_create.argtypes = [P, P, C.c_int32, C.c_int32, P, C.c_int32, C.POINTER(GenerateParams),
                                       C.c_int32, C.POINTER(P)]
    lib.mgx_session_step.argtypes = [P, C.c_int32, C.POINTER(C.c_int32)]
    lib.mgx_session_remaining.argtypes = [P]
    lib.mgx_session_finish.argtypes = [P, P, P, P, C.POINTER(GenerateReport)]
    lib.mgx_session_destroy.argtypes = [P]
    lib.mgx_session_destroy.restype = None
    lib.mgx_session_profile.argtypes = [P, C.c_int32]
    lib.mgx_session_profile_read.argtypes = [P, C.c_int32, C.POINTER(C.c_double), C.POINTER(C.c_double),
                                             C.POINTER(C.c_int32)]
    lib.mgx_session_hip_stream.restype = P
    lib.mgx_session_hip_stream.argtypes = [P]
    lib.mgx_batch_create.argtypes = [P, C.POINTER(BatchRequest), C.c_int32, C.c_int32, C.c_int32, C.c_int32,
                                     C.POINTER(P)]
    lib.mgx_batch_finish.argtypes = [P, C.c_int32, P, P, P, C.POINTER(GenerateReport)]
    lib.mgx_session_requests.argtypes = [P]
    lib.mgx_gguf_open.argtypes = [C.c_char_p, C.POINTER(P)]
    lib.mgx_gguf_close.argtypes = [P]
    lib.mgx_gguf_close.restype = None
    lib.mgx_gguf_tensor_count.argtypes = [P]
    lib.mgx_gguf_tensor.argtypes = [P, C.c_int32, C.POINTER(Tensor)]
    lib.mgx_gguf_find_tensor.argtypes = [P, C.c_char_p, C.POINTER(Tensor)]
    lib.mgx_gguf_u32.argtypes = [P, C.c_char_p, C.POINTER(C.c_uint32)]
    lib.mgx_gguf_f32.argtypes = [P, C.c_char_p, C.POINTER(C.c_float)]
    lib.mgx_gguf_string.argtypes = [P, C.c_char_p, C.c_char_p, C.c_uint64, C.POINTER(C.c_uint64)]
    lib.mgx_gguf_lm_config.argtypes = [P, C.POINTER(LmConfig)]
    lib.mgx_model_create_from_gguf.argtypes = [P, C.POINTER(P)]
    lib.mgx_model_set_adapters_from_gguf.argtypes = [P, P, P, C.c_float]
    lib.mgx_server_create.argtypes = [P, C.POINTER(ServerConfig), C.POINTER(P)]
    lib.mgx_server_generate.argtypes = [P, P, C.c_int32, C.c_int32, P, C.c_int32, C.POINTER(GenerateParams),
                                        PROGRESS_FN, P, P, P, P, C.POINTER(GenerateReport)]
    lib.mgx_server_stats.argtypes = [P, C.POINTER(ServerCounters)]
    lib.mgx_server_destroy.argtypes = [P]
    lib.mgx_server_destroy.restype = None
    lib.mgx_t5_create.argtypes = [C.POINTER(T5Config), C.POINTER(Tensor), C.c_int32, C.POINTER(P)]
    lib.mgx_gguf_t5_config.argtypes = [P, C.POINTER(T5Config)]
    lib.mgx_t5_create_from_gguf.argtypes = [P, C.POINTER(P)]
    lib.mgx_t5_encode.argtypes = [P, P, C.c_int32, P]
    lib.mgx_t5_destroy.argtypes = [P]
    lib.mgx_t5_destroy.restype = None
    lib.mgx_t5_relative_bucket.argtypes = [C.c_int32, C.c_int32, C.c_int32]
    lib.mgx_codec_create.argtypes = [C.POINTER(CodecConfig), C.POINTER(Tensor), C.c_int32, C.POINTER(P)]
    lib.mgx_gguf_codec_config.argtypes = [P, C.POINTER(CodecConfig)]
    lib.mgx_codec_create_from_gguf.argtypes = [P, C.POINTER(P)]
    lib.mgx_codec_decode.argtypes = [P, P, C.c_int32, P]
    lib.mgx_codec_decode_latent.argtypes = [P, P, C.c_int32, P]
    lib.mgx_codec_destroy.argtypes = [P]
    lib.mgx_codec_destroy.restype = None
    if path is None:
        _lib = lib
    return lib


def _check(lib, rc):
    if rc != 0:
        raise MgxError(rc, lib.mgx_last_error().decode())


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def use_guidance(cfg_coef, description_empty):
    return bool(load().mgx_use_guidance(cfg_coef, 1 if description_empty else 0))


def _tensor_array(tensors, names):
    """(name, ggml type, ne0, ne1, bytes) tuples as an mgx_tensor array; names keeps the
    encoded names alive."""
    arr = (Tensor * len(tensors))()
    for i, (name, ttype, ne0, ne1, data) in enumerate(tensors):
        b = name.encode()
        names.append(b)
        arr[i].name = b
        arr[i].type = ttype
        arr[i].ne[0], arr[i].ne[1], arr[i].ne[2], arr[i].ne[3] = ne0, ne1, 1, 1
        arr[i].data = data.ctypes.data
        arr[i].nbytes = data.nbytes
    return arr


def t5_relative_bucket(relative_position, num_buckets=32, max_distance=128):
    return load().mgx_t5_relative_bucket(int(relative_position), num_buckets, max_distance)


class Model:
    """mgx_model: the weights of one LM uploaded to the current HIP device."""

    def __init__(self, config, tensors):
        self.lib = load()
        self.config = config
        self._names = []
        arr = _tensor_array(tensors, self._names)
        h = C.c_void_p()
        _check(self.lib, self.lib.mgx_model_create(C.byref(config), arr, len(tensors), C.byref(h)))
        self.handle = h

    @classmethod
    def from_gguf(cls, gguf):
        """mgx_model_create_from_gguf: LmConfig::from + every tensor of an open Gguf."""
        m = cls.__new__(cls)
        m.lib = load()
        m.config = gguf.lm_config()
        h = C.c_void_p()
        _check(m.lib, m.lib.mgx_model_create_from_gguf(gguf.handle, C.byref(h)))
        m.handle = h
        return m

    def set_adapters_from_gguf(self, adapter, base=None, strength=1.0):
        """mgx_model_set_adapters_from_gguf: load_mg_lora on an open adapter Gguf."""
        _check(self.lib, self.lib.mgx_model_set_adapters_from_gguf(self.handle, adapter.handle,
                                                                   base.handle if base else None, strength))

    def set_adapters(self, adapters):
        """mgx_model_set_adapters. adapters: dicts with target, A [rank][in], B [out][rank],
        magnitude [out] or None, alpha, strength (rank is A's row count). [] detaches."""
        arr = (Adapter * max(1, len(adapters)))()
        keep = []
        for i, a in enumerate(adapters):
            A = np.ascontiguousarray(a["A"], np.float32)
            B = np.ascontiguousarray(a["B"], np.float32)
            m = a.get("magnitude")
            m = None if m is None else np.ascontiguousarray(m, np.float32)
            t = a["target"].encode()
            keep += [A, B, m, t]
            arr[i].target = t
            arr[i].A = A.ctypes.data
            arr[i].B = B.ctypes.data
            arr[i].magnitude = None if m is None else m.ctypes.data
            arr[i].rank = int(a.get("rank", A.shape[0]))
            arr[i].alpha = float(a["alpha"])
            arr[i].strength = float(a.get("strength", 1.0))
        _check(self.lib, self.lib.mgx_model_set_adapters(self.handle, arr if adapters else None, len(adapters)))

    def close(self):
        if self.handle:
            self.lib.mgx_model_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def generate(self, t5_hidden, prompt_codes, prompt_len, params, description_empty=False, step_logits=False):
        """mg_generate: returns (codes [n_q][T], first_logits [n_q][card], report, step_logits|None)."""
        c = self.config
        T = params.max_gen_len
        S = T + c.n_q
        start = prompt_len + 1
        codes = np.zeros((c.n_q, T), np.int32)
        first = np.zeros((c.n_q, c.card), np.float32)
        steps = np.zeros((S - start, c.n_q, c.card), np.float32) if step_logits else None
        rep = GenerateReport()
        t5 = np.ascontiguousarray(t5_hidden, np.float32)
        prompt = np.ascontiguousarray(prompt_codes, np.int32) if prompt_len else None
        _check(self.lib, self.lib.mgx_generate(self.handle, _ptr(t5), t5.shape[0], 1 if description_empty else 0,
                                               _ptr(prompt), prompt_len, C.byref(params), _ptr(codes), _ptr(first),
                                               _ptr(steps), C.byref(rep)))
        return codes, first, rep, steps


class Gguf:
    """mgx_gguf: a GGUF file mapped read-only (GgufModel without ggml)."""

    def __init__(self, path):
        self.lib = load()
        h = C.c_void_p()
        _check(self.lib, self.lib.mgx_gguf_open(str(path).encode(), C.byref(h)))
        self.handle = h

    def tensors(self):
        """[(name, ggml type, ne (4), nbytes, bytes)] in file order."""
        out = []
        for i in range(self.lib.mgx_gguf_tensor_count(self.handle)):
            t = Tensor()
            _check(self.lib, self.lib.mgx_gguf_tensor(self.handle, i, C.byref(t)))
            out.append((t.name.decode(), t.type, tuple(t.ne), t.nbytes, C.string_at(t.data, t.nbytes)))
        return out

    def u32(self, key):
        v = C.c_uint32()
        _check(self.lib, self.lib.mgx_gguf_u32(self.handle, key.encode(), C.byref(v)))
        return v.value

    def f32(self, key):
        v = C.c_float()
        _check(self.lib, self.lib.mgx_gguf_f32(self.handle, key.encode(), C.byref(v)))
        return v.value

    def string(self, key):
        n = C.c_uint64()
        _check(self.lib, self.lib.mgx_gguf_string(self.handle, key.encode(), None, 0, C.byref(n)))
        buf = C.create_string_buffer(n.value + 1)
        _check(self.lib, self.lib.mgx_gguf_string(self.handle, key.encode(), buf, n.value + 1, None))
        return buf.value.decode()

    def lm_config(self):
        c = LmConfig()
        _check(self.lib, self.lib.mgx_gguf_lm_config(self.handle, C.byref(c)))
        return c

    def codec_config(self):
        c = CodecConfig()
        _check(self.lib, self.lib.mgx_gguf_codec_config(self.handle, C.byref(c)))
        return c

    def t5_config(self):
        c = T5Config()
        _check(self.lib, self.lib.mgx_gguf_t5_config(self.handle, C.byref(c)))
        return c

    def close(self):
        if self.handle:
            self.lib.mgx_gguf_close(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Stream:
    """mgx_stream: one Decoder (KV cache + projected memory) over a Model."""

    def __init__(self, model, capacity, n_seq, t5_hidden=None, cross_attention=True):
        self.lib = model.lib
        self.model = model
        self.n_seq = n_seq
        t5 = None if t5_hidden is None else np.ascontiguousarray(t5_hidden, np.float32)
        h = C.c_void_p()
        _check(self.lib, self.lib.mgx_stream_create(model.handle, capacity, n_seq, _ptr(t5),
                                                    0 if t5 is None else t5.shape[0], 1 if cross_attention else 0,
                                                    C.byref(h)))
        self.handle = h

    def forward(self, ids):
        """ids [n_q][n_tokens] -> logits [n_seq][n_q][card] of the last position."""
        c = self.model.config
        ids = np.ascontiguousarray(ids, np.int32)
        out = np.zeros((self.n_seq, c.n_q, c.card), np.float32)
        _check(self.lib, self.lib.mgx_forward(self.handle, _ptr(ids), ids.shape[1], _ptr(out)))
        return out

    def used(self):
        return self.lib.mgx_stream_used(self.handle)

    def forwards(self):
        return self.lib.mgx_stream_forwards(self.handle)

    def cache_bytes(self):
        return self.lib.mgx_stream_cache_bytes(self.handle)

    def reset(self):
        _check(self.lib, self.lib.mgx_stream_reset(self.handle))

    def close(self):
        if self.handle:
            self.lib.mgx_stream_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Session:
    """mgx_session: mg_generate cut into resumable pieces (prefill first, then decodes)."""

    def __init__(self, model, t5_hidden, prompt_codes, prompt_len, params, description_empty=False,
                 keep_step_logits=False):
        self.lib = model.lib
        self.model = model
        self.params = params
        self.prompt_len = prompt_len
        self.keep = keep_step_logits
        t5 = np.ascontiguousarray(t5_hidden, np.float32)
        prompt = np.ascontiguousarray(prompt_codes, np.int32) if prompt_len else None
        h = C.c_void_p()
        _check(self.lib, self.lib.mgx_session_create(model.handle, _ptr(t5), t5.shape[0], 1 if description_empty else 0,
                                                     _ptr(prompt), prompt_len, C.byref(params),
                                                     1 if keep_step_logits else 0, C.byref(h)))
        self.handle = h

    def step(self, n):
        done = C.c_int32()
        _check(self.lib, self.lib.mgx_session_step(self.handle, n, C.byref(done)))
        return done.value

    def remaining(self):
        return self.lib.mgx_session_remaining(self.handle)

    def profile(self, every):
        _check(self.lib, self.lib.mgx_session_profile(self.handle, every))

    def profile_read(self, kind):
        ms, by, n = C.c_double(), C.c_double(), C.c_int32()
        _check(self.lib, self.lib.mgx_session_profile_read(self.handle, kind, C.byref(ms), C.byref(by), C.byref(n)))
        return ms.value, by.value, n.value

    def hip_stream(self):
        return self.lib.mgx_session_hip_stream(self.handle)

    def finish(self):
        c = self.model.config
        T = self.params.max_gen_len
        S = T + c.n_q
        start = self.prompt_len + 1
        codes = np.zeros((c.n_q, T), np.int32)
        first = np.zeros((c.n_q, c.card), np.float32)
        steps = np.zeros((S - start, c.n_q, c.card), np.float32) if self.keep else None
        rep = GenerateReport()
        _check(self.lib, self.lib.mgx_session_finish(self.handle, _ptr(codes), _ptr(first), _ptr(steps),
                                                     C.byref(rep)))
        return codes, first, rep, steps

    def close(self):
        if self.handle:
            self.lib.mgx_session_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Batch(Session):
    """mgx_batch_*: several requests decoded in lockstep, one KV cache column set each.

    requests: dicts with t5 [n_ctx][cond_dim], prompt [n_q][prompt_len], params
    (GenerateParams) and optionally description_empty."""

    def __init__(self, model, requests, prompt_len, keep_step_logits=False):
        self.lib = model.lib
        self.model = model
        self.params = requests[0]["params"]
        self.prompt_len = prompt_len
        self.keep = keep_step_logits
        self.n = len(requests)
        arr = (BatchRequest * self.n)()
        self._keep = []
        n_ctx = None
        for i, r in enumerate(requests):
            t5 = np.ascontiguousarray(r["t5"], np.float32)
            n_ctx = t5.shape[0] if n_ctx is None else n_ctx
            prompt = np.ascontiguousarray(r["prompt"], np.int32) if prompt_len else None
            self._keep += [t5, prompt]
            arr[i].t5_hidden = t5.ctypes.data
            arr[i].description_empty = 1 if r.get("description_empty") else 0
            arr[i].prompt_codes = None if prompt is None else prompt.ctypes.data
            arr[i].params = r["params"]
        h = C.c_void_p()
        _check(self.lib, self.lib.mgx_batch_create(model.handle, arr, self.n, n_ctx, prompt_len,
                                                   1 if keep_step_logits else 0, C.byref(h)))
        self.handle = h

    def requests(self):
        return self.lib.mgx_session_requests(self.handle)

    def finish(self, request=0):
        c = self.model.config
        T = self.params.max_gen_len
        S = T + c.n_q
        start = self.prompt_len + 1
        codes = np.zeros((c.n_q, T), np.int32)
        first = np.zeros((c.n_q, c.card), np.float32)
        steps = np.zeros((S - start, c.n_q, c.card), np.float32) if self.keep else None
        rep = GenerateReport()
        _check(self.lib, self.lib.mgx_batch_finish(self.handle, request, _ptr(codes), _ptr(first), _ptr(steps),
                                                   C.byref(rep)))
        return codes, first, rep, steps


class Server:
    """mgx_server_*: concurrent requests sharing one batched decode. generate() blocks the calling
    thread until its request is done (ctypes releases the GIL meanwhile, so Python threads run
    requests concurrently)."""

    def __init__(self, model, slots, max_gen_len, max_ctx=64, guided=True, keep_step_logits=False,
                 steps_per_round=0):
        self.lib = model.lib
        self.model = model
        self.keep = keep_step_logits
        cfg = ServerConfig(slots, 1 if guided else 0, max_gen_len, max_ctx, 1 if keep_step_logits else 0,
                           steps_per_round)
        h = C.c_void_p()
        _check(self.lib, self.lib.mgx_server_create(model.handle, C.byref(cfg), C.byref(h)))
        self.handle = h

    def generate(self, t5_hidden, prompt_codes, prompt_len, params, description_empty=False, step_logits=False,
                 progress=None):
        """As Model.generate; progress(done, total) is called from the server's worker thread."""
        c = self.model.config
        T = params.max_gen_len
        S = T + c.n_q
        start = prompt_len + 1
        codes = np.zeros((c.n_q, T), np.int32)
        first = np.zeros((c.n_q, c.card), np.float32)
        steps = np.zeros((S - start, c.n_q, c.card), np.float32) if step_logits else None
        rep = GenerateReport()
        t5 = np.ascontiguousarray(t5_hidden, np.float32)
        prompt = np.ascontiguousarray(prompt_codes, np.int32) if prompt_len else None
        cb = PROGRESS_FN(lambda user, done, total: progress(done, total)) if progress else PROGRESS_FN()
        _check(self.lib, self.lib.mgx_server_generate(self.handle, _ptr(t5), t5.shape[0],
                                                      1 if description_empty else 0, _ptr(prompt), prompt_len,
                                                      C.byref(params), cb, None, _ptr(codes), _ptr(first),
                                                      _ptr(steps), C.byref(rep)))
        return codes, first, rep, steps

    def counters(self):
        out = ServerCounters()
        _check(self.lib, self.lib.mgx_server_stats(self.handle, C.byref(out)))
        return {k: getattr(out, k) for k, _ in ServerCounters._fields_}

    def close(self):
        if getattr(self, "handle", None):
            self.lib.mgx_server_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class T5:
    """mgx_t5: the T5-base encoder resident on the current HIP device."""

    def __init__(self, config, tensors):
        self.lib = load()
        self.config = config
        names = []
        arr = _tensor_array(tensors, names)
        h = C.c_void_p()
        _check(self.lib, self.lib.mgx_t5_create(C.byref(config), arr, len(tensors), C.byref(h)))
        self.handle = h

    @classmethod
    def from_gguf(cls, gguf):
        t = cls.__new__(cls)
        t.lib = load()
        t.config = gguf.t5_config()
        h = C.c_void_p()
        _check(t.lib, t.lib.mgx_t5_create_from_gguf(gguf.handle, C.byref(h)))
        t.handle = h
        return t

    def encode(self, ids):
        """last_hidden_state [n_tokens][dim] of token ids [n_tokens]."""
        ids = np.ascontiguousarray(ids, np.int32)
        out = np.zeros((ids.size, self.config.dim), np.float32)
        _check(self.lib, self.lib.mgx_t5_encode(self.handle, _ptr(ids), ids.size, _ptr(out)))
        return out

    def close(self):
        if getattr(self, "handle", None):
            self.lib.mgx_t5_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Codec:
    """mgx_codec: the EnCodec decoder resident on the current HIP device. tensors: (name, ggml
    type, ne list, bytes) -- the codec's tensors are up to 3-D."""

    def __init__(self, config, tensors):
        self.lib = load()
        self.config = config if isinstance(config, CodecConfig) else CodecConfig.of(config)
        names = []
        arr = (Tensor * len(tensors))()
        for i, (name, ttype, ne, data) in enumerate(tensors):
            b = name.encode()
            names.append(b)
            arr[i].name, arr[i].type = b, ttype
            for d in range(4):
                arr[i].ne[d] = ne[d] if d < len(ne) else 1
            arr[i].data, arr[i].nbytes = data.ctypes.data, data.nbytes
        h = C.c_void_p()
        _check(self.lib, self.lib.mgx_codec_create(C.byref(self.config), arr, len(tensors), C.byref(h)))
        self.handle = h

    @classmethod
    def from_gguf(cls, gguf):
        k = cls.__new__(cls)
        k.lib = load()
        k.config = gguf.codec_config()
        h = C.c_void_p()
        _check(k.lib, k.lib.mgx_codec_create_from_gguf(gguf.handle, C.byref(h)))
        k.handle = h
        return k

    def decode(self, codes):
        """codes [n_q][frames] -> audio [channels][frames * hop_length]."""
        codes = np.ascontiguousarray(codes, np.int32)
        frames = codes.shape[1]
        out = np.zeros((self.config.channels, frames * self.config.hop_length), np.float32)
        _check(self.lib, self.lib.mgx_codec_decode(self.handle, _ptr(codes), frames, _ptr(out)))
        return out

    def decode_latent(self, latent):
        latent = np.ascontiguousarray(latent, np.float32)
        frames = latent.shape[1]
        out = np.zeros((self.config.channels, frames * self.config.hop_length), np.float32)
        _check(self.lib, self.lib.mgx_codec_decode_latent(self.handle, _ptr(latent), frames, _ptr(out)))
        return out

    def close(self):
        if getattr(self, "handle", None):
            self.lib.mgx_codec_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
