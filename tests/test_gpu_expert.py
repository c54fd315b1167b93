"""One SwiGLU expert at batch 1 (fdm_expert_ffn), down projection as Q4_K
and as Q6_K, against the oracle (bit-exact dequant + float64 dots).
Tolerance 1e-3 relative L2."""
import numpy as np
import pytest

from tests._helpers import empty_f32, rel_l2, say, to_dev, to_host

pytestmark = pytest.mark.gpu
TOL = 1e-3


@pytest.mark.parametrize("q6", [False, True])
def test_expert_ffn(fdm, oracle, q6):
    say(f"expert_ffn q6={q6}")
    blob = oracle.synth_expert(5, down_is_q6=q6)
    x = oracle.synth_normal(7168, 0.0, 1.0, 6)
    out, act = empty_f32(7168), empty_f32(2048)
    size = fdm.EXPERT_Q6K_BYTES if q6 else fdm.EXPERT_Q4K_BYTES
    fdm.expert_ffn(to_dev(blob), size, to_dev(x), out, act)
    want, _, _, want_act = oracle.expert_ffn(blob, q6, x, with_intermediates=True)
    e_act, e_out = rel_l2(to_host(act), want_act), rel_l2(to_host(out), want)
    print(f"act rel_l2={e_act:.3e} out rel_l2={e_out:.3e}")
    assert e_act <= TOL and e_out <= TOL


@pytest.mark.parametrize("q6", [False, True])
def test_expert_fp32_grade(fdm, oracle, q6):
    """Against float64, the expert's error stays within 4x that of the
    reference's fp32 arithmetic (oracle.expert_ffn_f32)."""
    say(f"expert_ffn fp32 grade q6={q6}")
    blob = oracle.synth_expert(15, down_is_q6=q6)
    x = oracle.synth_normal(7168, 0.0, 1.0, 16)
    out = empty_f32(7168)
    size = fdm.EXPERT_Q6K_BYTES if q6 else fdm.EXPERT_Q4K_BYTES
    fdm.expert_ffn(to_dev(blob), size, to_dev(x), out)
    want = oracle.expert_ffn(blob, q6, x).astype(np.float64)
    e_got = rel_l2(to_host(out), want)
    e_f32 = rel_l2(oracle.expert_ffn_f32(blob, q6, x), want)
    print(f"rel_l2 {e_got:.3e} (fp32 restatement {e_f32:.3e})")
    assert e_got <= 4 * e_f32


def test_expert_rejects_bad_size(fdm, oracle):
    blob = to_dev(np.zeros(16, np.uint8))
    with pytest.raises(fdm.FdmError):
        fdm.expert_ffn(blob, 12345, empty_f32(7168), empty_f32(7168))
