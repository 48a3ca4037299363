"""Python access to the MI355X MusicGen LM decode library (libmgx.so) for tests and the
benchmark: ctypes bindings over the C ABI in include/mgx.h and a seeded synthetic-model
builder. The library itself is C/HIP; nothing here computes on the host."""
from .lib import (Batch, Gguf, Model, Server, Session, Stream, GenerateParams, GenerateReport, LmConfig, MgxError, load,
                  use_guidance)
from .synth import SHAPES, SyntheticModel, make_config, synth_adapters, synth_codes, synth_memory

__all__ = ["Batch", "Gguf", "Model", "Server", "Session", "Stream", "GenerateParams", "GenerateReport", "LmConfig", "MgxError", "load",
           "use_guidance", "SHAPES", "SyntheticModel", "make_config", "synth_adapters", "synth_codes",
           "synth_memory"]
