"""The GGUF reader (mgx_gguf_*) on the host: files written by mgx.gguf, read back through the C
ABI, against GgufModel / LmConfig::from (src/gguf_model.h:241-414, src/mg/lm.h:60-90)."""
import struct

import numpy as np
import pytest

import mgx
from mgx import gguf as G
from tests import helpers as H


def lm_file(tmp_path, shape="tiny", wtype=8, seed=3, kv=None, name="m.gguf"):
    m = H.model(shape, wtype, seed)
    p = tmp_path / name
    G.write_lm(str(p), m, kv=kv)
    return m, p


@pytest.mark.parametrize("wtype", [8, 2, 1, 0])
def test_lm_round_trip(tmp_path, wtype):
    m, p = lm_file(tmp_path, wtype=wtype)
    g = mgx.Gguf(p)
    c, want = g.lm_config(), m.config
    for f in ("dim", "layers", "heads", "head_dim", "ff_dim", "cond_dim", "n_q", "card", "special_token_id",
              "pos_denominator", "max_period", "norm_eps", "cfg_coef"):
        assert getattr(c, f) == getattr(want, f), f
    got = g.tensors()
    assert [t[0] for t in got] == [t[0] for t in m.tensors]
    for (name, ttype, ne, nbytes, data), (n2, t2, ne0, ne1, raw) in zip(got, m.tensors):
        assert ttype == t2 and ne == (ne0, ne1, 1, 1) and data == raw.tobytes() and nbytes == raw.nbytes, name
    assert g.string("general.architecture") == "ac-musicgen-lm"
    g.close()


def test_reference_fixture_metadata(tmp_path):
    """The tiny LM of tests/mg_train_cli_test.py:28-42 (F32, dim 8, card 11): LmConfig::from's
    values and the converter's tensor names; its head_dim 4 is below what the decode kernels take,
    so only the file layer is exercised."""
    rng = np.random.default_rng(77)
    shapes = {"lm.cond_proj.weight": (8, 6), "lm.cond_proj.bias": (8,), "lm.out_norm.weight": (8,),
              "lm.out_norm.bias": (8,)}
    for q in range(4):
        shapes[f"lm.emb.{q}.weight"] = (12, 8)
        shapes[f"lm.head.{q}.weight"] = (11, 8)
    for i in range(2):
        for norm in ("norm1", "norm_cross", "norm2"):
            shapes[f"lm.{i}.{norm}.weight"] = (8,)
            shapes[f"lm.{i}.{norm}.bias"] = (8,)
        for stem, shape in [("self.qkv", (24, 8)), ("self.out", (8, 8)), ("cross.q", (8, 8)), ("cross.kv", (16, 8)),
                            ("cross.out", (8, 8)), ("ff.0", (16, 8)), ("ff.2", (8, 16))]:
            shapes[f"lm.{i}.{stem}.weight"] = shape
    tensors = {k: rng.normal(0, .15, s).astype(np.float32) for k, s in shapes.items()}
    kv = [("general.architecture", G.STR, "ac-musicgen-lm"), ("general.name", G.STR, "MusicGen CLI fixture"),
          ("ac.architecture", G.STR, "audiocraft"), ("ac.format_version", G.U32, 1),
          ("ac.lm.family", G.STR, "musicgen"), ("ac.lm.dim", G.U32, 8), ("ac.lm.layers", G.U32, 2),
          ("ac.lm.heads", G.U32, 2), ("ac.lm.head_dim", G.U32, 4), ("ac.lm.ff_dim", G.U32, 16),
          ("ac.lm.cond_dim", G.U32, 6), ("ac.lm.n_q", G.U32, 4), ("ac.lm.card", G.U32, 11),
          ("ac.lm.special_token_id", G.U32, 11), ("ac.lm.pos_denominator", G.U32, 3),
          ("ac.lm.max_period", G.F32, 10000.0), ("ac.lm.norm_eps", G.F32, 1e-5), ("ac.lm.cfg_coef", G.F32, 3.0),
          ("ac.lm.sample_rate", G.U32, 32000), ("ac.lm.max_duration", G.F32, 30.0)]
    p = tmp_path / "base.gguf"
    G.write(str(p), kv, [(k, 0, list(v.shape[::-1]), v) for k, v in tensors.items()])
    g = mgx.Gguf(p)
    c = g.lm_config()
    assert (c.dim, c.layers, c.heads, c.head_dim, c.ff_dim, c.cond_dim, c.n_q, c.card, c.special_token_id,
            c.pos_denominator) == (8, 2, 2, 4, 16, 6, 4, 11, 11, 3)
    assert (c.max_period, c.cfg_coef) == (10000.0, 3.0) and c.norm_eps == np.float32(1e-5)
    got = {t[0]: t for t in g.tensors()}
    for k, v in tensors.items():
        ne = tuple(list(v.shape[::-1]) + [1] * (4 - v.ndim))
        assert got[k][2] == ne and got[k][4] == v.tobytes(), k


def expect(path, text):
    with pytest.raises(mgx.MgxError) as e:
        g = mgx.Gguf(path)
        g.lm_config()
    assert text in str(e.value), str(e.value)


def test_lm_config_checks(tmp_path):
    """LmConfig::from's throws (lm.h:61-88), with the reference's messages."""
    c = H.model("tiny", 8, 3).config
    base = G.lm_kv(c)

    def with_kv(name, edit):
        kv = [e for e in base if e[0] != edit[0]] + ([edit] if edit[1] is not None else [])
        return lm_file(tmp_path, kv=kv, name=name)[1]

    expect(with_kv("a.gguf", ("ac.architecture", G.STR, "other")), "not an audiocraft GGUF")
    expect(with_kv("b.gguf", ("ac.format_version", G.U32, 2)), "unsupported audiocraft GGUF version")
    expect(with_kv("c.gguf", ("ac.lm.family", G.STR, "melodyflow")), "not a MusicGen LM GGUF")
    expect(with_kv("d.gguf", ("ac.lm.dim", None, None)), "missing key: ac.lm.dim")
    expect(with_kv("e.gguf", ("ac.lm.heads", G.U32, 3)), "LM dim does not equal heads * head_dim")
    expect(with_kv("f.gguf", ("ac.lm.special_token_id", G.U32, 7)), "special_token_id should be card")
    expect(with_kv("g.gguf", ("ac.lm.max_period", G.U32, 10000)), "key is not f32: ac.lm.max_period")
    expect(with_kv("h.gguf", ("ac.lm.sample_rate", None, None)), "missing key: ac.lm.sample_rate")


def test_file_checks(tmp_path):
    """Malformed files fail with a message, never a crash: magic, version, truncation (load_gguf's
    short-read check, gguf_model.h:384-389), misalignment, unknown tensor types, duplicates."""
    m, p = lm_file(tmp_path)
    raw = p.read_bytes()
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"GGUX" + raw[4:])
    expect(bad, "not a GGUF file")
    bad.write_bytes(raw[:4] + struct.pack("<I", 1) + raw[8:])
    expect(bad, "unsupported GGUF version 1")
    bad.write_bytes(raw[:len(raw) - 100])
    expect(bad, "short read while loading tensor lm.head.3.weight")
    bad.write_bytes(raw[:2000])
    expect(bad, "runs past the end of the file")
    bad.write_bytes(b"")
    expect(bad, "empty file")
    expect(tmp_path / "missing.gguf", "failed to open")
    # GGUF v2 has the same layout for these fields and is accepted
    p2 = tmp_path / "v2.gguf"
    G.write(str(p2), G.lm_kv(m.config), [(n, t, [a, b] if b > 1 else [a], d) for n, t, a, b, d in m.tensors], version=2)
    assert mgx.Gguf(p2).lm_config().dim == m.config.dim
    one = [("x", 0, [4], np.zeros(4, np.float32))]
    G.write(str(bad), [("k", G.U32, 1), ("k", G.U32, 2)], one)
    expect(bad, "duplicate key k")
    G.write(str(bad), [], [("x", 0, [4], np.zeros(4, np.float32)), ("x", 0, [4], np.zeros(4, np.float32))])
    expect(bad, "duplicate tensor x")
    G.write(str(bad), [], [("x", 13, [32], np.zeros(32, np.uint8))])
    expect(bad, "unsupported type 13")
    G.write(str(bad), [], [("x", 8, [48], np.zeros(34 * 2, np.uint8))])
    expect(bad, "split a block")
    G.write(str(bad), [("general.alignment", G.U32, 48)], one)
    expect(bad, "bad alignment")
