"""A minimal GGUF v3 writer for synthetic MusicGen LM and adapter files.

It writes what tools/convert_musicgen_lm.py:148-222 and the reference's adapter writer put in a
file -- general.architecture, the ac.* keys (src/mg/lm.h:60-90, src/ac/lora.h:113-150) and the
tensors in ggml block layouts -- so the library's GGUF reader can be tested against files whose
every byte is known. Layout (the public GGUF v3 format): magic, version, tensor and key counts,
key/values, tensor infos (name, dims, ggml type, offset), padding to the alignment, data."""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
ALIGN = 32


def _s(b, text):
    raw = text.encode()
    b += struct.pack("<Q", len(raw)) + raw


def _value(b, vtype, v):
    fmt = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q",
           I64: "<q", F64: "<d"}
    if vtype == STR:
        _s(b, v)
    elif vtype == ARR:
        etype, items = v
        b += struct.pack("<IQ", etype, len(items))
        for it in items:
            _value(b, etype, it)
    else:
        b += struct.pack(fmt[vtype], v)


def write(path, kv, tensors, alignment=ALIGN, version=3):
    """kv: list of (key, gguf type, value) -- arrays as (element type, list); tensors: list of
    (name, ggml type, ne list (ne[0] contiguous), raw bytes as a uint8 array)."""
    b = bytearray(b"GGUF")
    b += struct.pack("<IQQ", version, len(tensors), len(kv))
    for key, vtype, v in kv:
        _s(b, key)
        b += struct.pack("<I", vtype)
        _value(b, vtype, v)
    tensors = [(n, t, ne, np.ascontiguousarray(d).view(np.uint8).reshape(-1)) for n, t, ne, d in tensors]
    offs, off = [], 0
    for name, ttype, ne, data in tensors:
        _s(b, name)
        b += struct.pack("<I", len(ne))
        for n in ne:
            b += struct.pack("<q", int(n))
        b += struct.pack("<IQ", ttype, off)
        offs.append(off)
        off += (len(data) + alignment - 1) // alignment * alignment
    b += bytes((-len(b)) % alignment)
    for (name, ttype, ne, data), o in zip(tensors, offs):
        raw = data.tobytes()
        b += raw + bytes((-len(raw)) % alignment)
    with open(path, "wb") as f:
        f.write(b)


def lm_kv(config, name="synthetic MusicGen LM", sample_rate=32000, max_duration=30.0):
    """The LM keys convert_musicgen_lm.py:149-173 writes, from an LmConfig."""
    c = config
    return [("general.architecture", STR, "ac-musicgen-lm"), ("ac.architecture", STR, "audiocraft"),
            ("ac.format_version", U32, 1), ("ac.lm.family", STR, "musicgen"), ("ac.lm.dim", U32, c.dim),
            ("ac.lm.layers", U32, c.layers), ("ac.lm.heads", U32, c.heads), ("ac.lm.head_dim", U32, c.head_dim),
            ("ac.lm.ff_dim", U32, c.ff_dim), ("ac.lm.cond_dim", U32, c.cond_dim), ("ac.lm.n_q", U32, c.n_q),
            ("ac.lm.card", U32, c.card), ("ac.lm.special_token_id", U32, c.special_token_id),
            ("ac.lm.delays", ARR, (I32, list(range(c.n_q)))), ("ac.lm.max_period", F32, c.max_period),
            ("ac.lm.pos_denominator", U32, c.pos_denominator), ("ac.lm.norm_eps", F32, c.norm_eps),
            ("ac.lm.cfg_coef", F32, c.cfg_coef), ("ac.lm.sample_rate", U32, sample_rate),
            ("ac.lm.max_duration", F32, max_duration), ("ac.lm.activation", STR, "gelu_erf"),
            ("general.name", STR, name)]


def write_lm(path, model, name="synthetic MusicGen LM", kv=None):
    """A SyntheticModel (list of (name, type, ne0, ne1, bytes)) as an LM GGUF file."""
    write(path, kv if kv is not None else lm_kv(model.config, name),
          [(n, t, [ne0, ne1] if ne1 > 1 else [ne0], data) for n, t, ne0, ne1, data in model.tensors])


def write_adapter(path, adapters, base_name=None, kv_extra=()):
    """Adapter dicts (target, A [rank][in], B [out][rank], magnitude or None, rank, alpha) as an
    "ac-musicgen-lora" file: stem.lora_A ggml [in, rank], stem.lora_B [rank, out],
    stem.magnitude [out] (lora.h:125-150)."""
    a0 = adapters[0]
    dora = a0.get("magnitude") is not None
    kv = [("general.architecture", STR, "ac-musicgen-lora"), ("ac.lora.version", U32, 1),
          ("ac.lora.rank", U32, int(a0["rank"])), ("ac.lora.alpha", F32, float(a0["alpha"])),
          ("ac.lora.type", STR, "dora-rows" if dora else "lora")]
    if base_name is not None:
        kv.append(("ac.lora.base_name", STR, base_name))
    kv += list(kv_extra)
    ts = []
    for a in adapters:
        A = np.ascontiguousarray(a["A"], np.float32)
        B = np.ascontiguousarray(a["B"], np.float32)
        ts.append((a["target"] + ".lora_A", 0, [A.shape[1], A.shape[0]], A))
        ts.append((a["target"] + ".lora_B", 0, [B.shape[1], B.shape[0]], B))
        if dora:
            m = np.ascontiguousarray(a["magnitude"], np.float32)
            ts.append((a["target"] + ".magnitude", 0, [m.shape[0]], m))
    write(path, kv, ts)


def t5_kv(config, max_length=256, weight_type="F16"):
    """The encoder keys tools/convert_t5.py:67-81 writes (tokenizer keys left out)."""
    c = config
    return [("general.architecture", STR, "ac-t5"), ("ac.t5.dim", U32, c.dim), ("ac.t5.layers", U32, c.layers),
            ("ac.t5.heads", U32, c.heads), ("ac.t5.head_dim", U32, c.head_dim),
            ("ac.t5.intermediate", U32, c.intermediate), ("ac.t5.vocab", U32, c.vocab),
            ("ac.t5.relative_buckets", U32, c.relative_buckets),
            ("ac.t5.relative_max_distance", U32, c.relative_max_distance), ("ac.t5.eps", F32, c.eps),
            ("ac.t5.max_length", U32, max_length), ("ac.t5.weight_type", STR, weight_type)]


def write_t5(path, model, kv=None):
    """A SyntheticT5 as a T5 encoder GGUF file."""
    write(path, kv if kv is not None else t5_kv(model.config),
          [(n, t, [ne0, ne1] if ne1 > 1 else [ne0], data) for n, t, ne0, ne1, data in model.tensors])


def codec_kv(cfg):
    """The codec keys tools/convert_seanet.py:395-415 writes, from a SeanetConfig-like dict."""
    kv = [("general.architecture", STR, "ac-seanet"), ("ac.architecture", STR, "audiocraft"),
          ("ac.format_version", U32, 1), ("ac.codec.quantizer", STR, cfg.get("quantizer", "rvq")),
          ("ac.codec.activation", STR, cfg.get("activation", "ELU")), ("ac.codec.channels", U32, cfg["channels"]),
          ("ac.codec.n_filters", U32, cfg["n_filters"]), ("ac.codec.n_residual_layers", U32, cfg["n_residual_layers"]),
          ("ac.codec.ratios", ARR, (I32, list(cfg["ratios"]))), ("ac.codec.kernel_size", U32, cfg["kernel_size"]),
          ("ac.codec.residual_kernel_size", U32, cfg["residual_kernel_size"]),
          ("ac.codec.last_kernel_size", U32, cfg["last_kernel_size"]),
          ("ac.codec.dilation_base", U32, cfg["dilation_base"]), ("ac.codec.compress", U32, cfg["compress"]),
          ("ac.codec.lstm_layers", U32, cfg["lstm_layers"]), ("ac.codec.latent_dim", U32, cfg["latent_dim"]),
          ("ac.codec.encoder_dim", U32, cfg["encoder_dim"]), ("ac.codec.sample_rate", U32, cfg["sample_rate"]),
          ("ac.codec.hop_length", U32, cfg["hop_length"]), ("ac.codec.frame_rate", U32, cfg["frame_rate"]),
          ("ac.codec.weight_type", STR, "F32")]
    if cfg.get("quantizer", "rvq") == "rvq":
        kv += [("ac.codec.rvq_n_q", U32, cfg["rvq_n_q"]), ("ac.codec.rvq_bins", U32, cfg["rvq_bins"])]
    return kv


def write_codec(path, codec, kv=None):
    """A SyntheticCodec as a codec GGUF file."""
    write(path, kv if kv is not None else codec_kv(codec.config), codec.tensors)
