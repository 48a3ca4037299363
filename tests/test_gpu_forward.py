"""HIP decode step vs the oracle, bit for bit, through the C ABI (mgx_forward)."""
import numpy as np
import pytest

from tests import helpers as H

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def mgx():
    import mgx as M
    M.load()
    return M


@pytest.mark.parametrize("wtype", [8, 2, 1, 0])
def test_tiny_forward_matches_oracle(mgx, wtype):
    from oracle import cpu_ref as R
    m = H.model("tiny", wtype, 3)
    c = m.config
    t5 = H.memory(1, 5)
    ids = H.codes(2, 4, 12, c.card)
    gm = mgx.Model(c, m.tensors)
    gs = mgx.Stream(gm, 40, 2, t5, True)
    rd = R.RefDecoder(H.ref_model("tiny", wtype, 3), 40, 2, t5, True)
    print(f"tiny forward wtype={wtype}: prefill 8 then 4 steps", flush=True)
    got = gs.forward(ids[:, :8])
    want = rd.forward(ids[:, :8])
    assert np.array_equal(got, want), f"prefill logits differ: max {np.abs(got - want).max()}"
    for t in range(8, 12):
        got = gs.forward(ids[:, t:t + 1])
        want = rd.forward(ids[:, t:t + 1])
        assert np.array_equal(got, want), f"step {t}: max {np.abs(got - want).max()}"
    assert gs.used() == 12 and gs.forwards() == 5
