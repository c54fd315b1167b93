"""MLA attention of decode tokens on the device (fdm_attn_*; mla_forward,
infer.m:766-903) against the oracle over a growing KV cache: hidden after
each token within 1e-3 relative L2 of the float64 truth (attention part and
whole), positions in order and after a jump, the cache length counted, a
reset reproducing the first token bit for bit, and the errors."""
import numpy as np
import pytest

from tests._helpers import rel_l2, say, to_dev, to_host
from tests.mla_case import H, mla_weights

pytestmark = pytest.mark.gpu
TOL = 1e-3


@pytest.fixture(scope="module")
def attn_layer(fdm):
    w = mla_weights(903)
    say("attn_upload L=0")
    fdm.attn_upload(0, w, max_seq=64)
    yield w
    fdm.attn_release(0)


def test_attn_tokens_match_oracle(fdm, oracle, attn_layer):
    w = attn_layer
    fdm.attn_reset(0)
    cache = oracle.MlaCache(64)
    rng = np.random.default_rng(5)
    first = None
    for n, pos in enumerate([0, 1, 2, 3, 4, 5, 100]):
        hidden = rng.normal(0, 1, H).astype(np.float32)
        d = to_dev(hidden)
        say(f"attn_forward pos={pos}")
        fdm.attn_forward(0, d, pos)
        got = to_host(d)
        want = oracle.mla_forward(w, hidden, cache, pos)
        err = rel_l2(got, want.astype(np.float64))
        err_attn = rel_l2(got.astype(np.float64) - hidden, want.astype(np.float64) - hidden)
        print(f"pos {pos}: rel_l2 {err:.2e}, attention part {err_attn:.2e}")
        assert err <= TOL and err_attn <= TOL, pos
        assert fdm.attn_len(0) == n + 1
        if first is None:
            first = (hidden, got)
    fdm.attn_reset(0)
    assert fdm.attn_len(0) == 0
    d = to_dev(first[0])
    fdm.attn_forward(0, d, 0)
    assert np.array_equal(to_host(d).view(np.uint32), first[1].view(np.uint32))


def test_attn_errors(fdm, attn_layer):
    x = to_dev(np.zeros(H, np.float32))
    with pytest.raises(fdm.FdmError):
        fdm.attn_forward(9, x, 0)  # not resident
    with pytest.raises(fdm.FdmError):
        fdm.attn_forward(0, x, -1)
    fdm.attn_upload(9, attn_layer, max_seq=2)
    try:
        fdm.attn_forward(9, x, 0)
        fdm.attn_forward(9, x, 1)
        with pytest.raises(fdm.FdmError):
            fdm.attn_forward(9, x, 2)  # cache full
    finally:
        fdm.attn_release(9)
    with pytest.raises(fdm.FdmError):
        fdm.attn_upload(9, attn_layer, max_seq=0)
