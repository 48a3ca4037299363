"""Python access to the MI355X MusicGen LM decode library (libmgx.so) for tests and the
benchmark: ctypes bindings over the C ABI in include/mgx.h and a seeded synthetic-model
builder. The library itself is C/HIP; nothing here computes on the host."""
from .lib import (Batch, Codec, CodecConfig, GenerateParams, GenerateReport, Gguf, LmConfig, MgxError, Model, Server, Session, Stream,
                  T5, T5Config, load, t5_relative_bucket, use_guidance)
from .synth import (CODEC_SHAPES, SHAPES, T5_SHAPES, SyntheticCodec, SyntheticModel, SyntheticT5, make_codec_config,
                    make_config, make_t5_config, synth_adapters,
                    synth_codes, synth_ids, synth_memory)

__all__ = ["Batch", "Codec", "CodecConfig", "CODEC_SHAPES", "SyntheticCodec", "make_codec_config", "GenerateParams", "GenerateReport", "Gguf", "LmConfig", "MgxError", "Model", "Server", "Session",
           "Stream", "T5", "T5Config", "load", "t5_relative_bucket", "use_guidance", "SHAPES", "T5_SHAPES",
           "SyntheticModel", "SyntheticT5", "make_config", "make_t5_config", "synth_adapters", "synth_codes",
           "synth_ids", "synth_memory"]
