"""Models and adapters loaded from GGUF files (mgx_model_create_from_gguf,
mgx_model_set_adapters_from_gguf) against the same tensors handed over in memory."""
import numpy as np
import pytest

from mgx import gguf as G
from mgx import synth
from tests import helpers as H

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def M():
    import mgx
    mgx.load()
    return mgx


@pytest.mark.parametrize("shape,wtype", [("tiny", 8), ("tiny", 2), ("tiny", 1), ("mini1536", 8)])
def test_model_from_gguf_generates_the_same(M, tmp_path, shape, wtype):
    print(f"gguf generate {shape} wtype={wtype}", flush=True)
    m = H.model(shape, wtype, 9)
    p = tmp_path / "lm.gguf"
    G.write_lm(str(p), m)
    g = M.Gguf(p)
    gm = M.Model.from_gguf(g)
    g.close()   # the weights were uploaded: the mapping is no longer needed
    c = m.config
    t5 = H.memory(9, synth.SHAPES[shape]["n_ctx"])
    prompt = H.codes(9, c.n_q, 6, c.card)
    params = M.GenerateParams(24, 1, 1.0, 250, 3.0, 9)
    a = gm.generate(t5, prompt, 6, params, step_logits=True)
    b = M.Model(c, m.tensors).generate(t5, prompt, 6, params, step_logits=True)
    assert np.array_equal(a[3], b[3]) and np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


@pytest.mark.parametrize("dora", [False, True])
def test_adapters_from_gguf(M, tmp_path, dora):
    print(f"gguf adapters dora={dora}", flush=True)
    m = H.model("tiny", 8, 3)
    c = m.config
    ads = synth.synth_adapters(c, rank=8, targets=("self.qkv", "cross.out", "ff.2"), dora=dora, alpha=12.0, seed=5)
    base_p, ad_p = tmp_path / "base.gguf", tmp_path / "ad.gguf"
    G.write_lm(str(base_p), m, name="tiny base")
    G.write_adapter(str(ad_p), ads, base_name="tiny base")
    t5 = H.memory(1, 5)
    ids = H.codes(2, c.n_q, 6, c.card)
    want_m = M.Model(c, m.tensors)
    want_m.set_adapters([dict(a, strength=0.8) for a in ads])
    want = M.Stream(want_m, 8, 2, t5, True).forward(ids)
    base, ad = M.Gguf(base_p), M.Gguf(ad_p)
    gm = M.Model.from_gguf(base)
    gm.set_adapters_from_gguf(ad, base, strength=0.8)
    got = M.Stream(gm, 8, 2, t5, True).forward(ids)
    assert np.array_equal(got, want)


def test_adapter_file_checks(M, tmp_path):
    """load_lora / load_mg_lora's throws (lora.h:113-176, 195-210)."""
    m = H.model("tiny", 8, 3)
    c = m.config
    base_p = tmp_path / "base.gguf"
    G.write_lm(str(base_p), m, name="tiny base")
    base = M.Gguf(base_p)
    gm = M.Model.from_gguf(base)
    good = synth.synth_adapters(c, rank=4, targets=("ff.0",), dora=True)

    def expect(path, text, **kw):
        with pytest.raises(M.MgxError) as e:
            gm.set_adapters_from_gguf(M.Gguf(path), base, **kw)
        assert text in str(e.value), str(e.value)

    p = tmp_path / "a.gguf"
    G.write(str(p), [("general.architecture", G.STR, "ac-melodyflow-lora")], [("x", 0, [4], np.zeros(4, np.float32))])
    expect(p, "not a MusicGen adapter")
    G.write_adapter(str(p), good, kv_extra=[])
    expect(p, "invalid adapter rank, alpha or strength", strength=float("nan"))
    G.write_adapter(str(p), [dict(good[0], target="lm.0.ff.1.weight")])
    expect(p, "missing tensor: lm.0.ff.1.weight")   # load_lora looks the base tensor up first
    bad = dict(good[0], A=np.zeros((4, c.dim // 2), np.float32))
    G.write_adapter(str(p), [bad])
    expect(p, "adapter shape mismatch: lm.0.ff.0.weight")
    G.write_adapter(str(p), good, base_name="another model")
    expect(p, "adapter base model name does not match")
    # a DoRA file missing a magnitude: incomplete
    A, B = good[0]["A"], good[0]["B"]
    G.write(str(p), [("general.architecture", G.STR, "ac-musicgen-lora"), ("ac.lora.version", G.U32, 1),
                     ("ac.lora.rank", G.U32, 4), ("ac.lora.alpha", G.F32, 4.0), ("ac.lora.type", G.STR, "dora-rows")],
            [("lm.0.ff.0.weight.lora_A", 0, [A.shape[1], 4], A), ("lm.0.ff.0.weight.lora_B", 0, [4, B.shape[0]], B)])
    expect(p, "missing tensor: lm.0.ff.0.weight.magnitude")
