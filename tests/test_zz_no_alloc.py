"""fdm_moe_forward_batched_noalloc: the batched decode step on the library's
fixed device scratch (it allocates nothing), against fdm_moe_forward_batched
on the same inputs.  Both run the same kernels on buffers of the same
shapes, so the outputs, the routing and the distinct-expert count must be
bit-identical.  Two no-allocation calls run back to back, the second with
fewer tokens (and on the digit-kernel path, T < FDM_BATCH_MFMA_MIN_T), so
a leftover of the first call in the shared scratch would show; sizes past
the scratch's limits are rejected.  That the call allocates nothing is
checked by capturing it into a HIP graph on a fresh stream in global
capture mode, where any allocation (a workspace for that stream included)
is refused and invalidates the capture."""
import numpy as np
import pytest

from tests._helpers import bits_equal_nan_class, empty_f32, say, to_dev, to_host

pytestmark = pytest.mark.gpu
K = 8


@pytest.fixture(scope="module", params=[False, True], ids=["q4k_down", "q6k_down"])
def layer(request, fdm):
    from flash_deepseek_amd.synthetic import make_layer
    L = 15 if request.param else 14
    say(f"building layer L={L} down_q6={request.param}")
    lay = make_layer(2100 + L, down_q6=request.param)
    fdm.attach_layer(L, lay.experts, lay.expert_size, lay.Wg, lay.bias, lay.shared)
    yield L
    fdm.release_layer(L)


def tokens(T, seed):
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((T, 7168), dtype=np.float32)
    H = rng.standard_normal((T, 7168), dtype=np.float32)
    return to_dev(X.ravel()), to_dev(H.ravel())


def step(fdm, fn, L, X, H, T):
    import torch
    out = empty_f32(T * 7168)
    idx = torch.empty(T * K, dtype=torch.int32, device="cuda")
    w = empty_f32(T * K)
    nd = torch.zeros(1, dtype=torch.int32, device="cuda")
    fn(L, X, H, T, K, out, idx, w, nd)
    return out, idx, w, nd


@pytest.mark.parametrize("T", [16, 3], ids=["mfma_path", "dot4_path"])
def test_noalloc_captures_in_a_graph(fdm, layer, T):
    """The property the entry point exists for: it allocates nothing.  The
    call is captured into a HIP graph on a fresh stream in global capture
    mode (hipMalloc, and so a stream workspace, is refused there and the
    capture fails).  Each replay, with eager work and synchronisations
    between replays, equals the eager fdm_moe_forward_batched bit for bit."""
    import torch
    L = layer
    X, H = tokens(T, 43 + T)
    say(f"moe_forward_batched (eager reference) L={L} T={T}")
    want = [to_host(t) for t in step(fdm, fdm.moe_forward_batched, L, X, H, T)]
    fdm.sync()
    out = empty_f32(T * 7168)
    idx = torch.empty(T * K, dtype=torch.int32, device="cuda")
    w = empty_f32(T * K)
    nd = torch.zeros(1, dtype=torch.int32, device="cuda")
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    say(f"capturing moe_forward_batched_noalloc L={L} T={T} on a fresh stream")
    with torch.cuda.graph(g, stream=s, capture_error_mode="global"):
        fdm.moe_forward_batched_noalloc(L, X, H, T, K, out, idx, w, nd, stream=s.cuda_stream)
    for r in range(3):
        # eager work on the outputs between replays: a replay must rewrite all of them
        out.fill_(float("nan"))
        idx.fill_(-1)
        w.fill_(float("nan"))
        nd.fill_(-1)
        torch.cuda.synchronize()
        say(f"replay {r} L={L} T={T}")
        g.replay()
        torch.cuda.synchronize()
        got = [to_host(t) for t in (out, idx, w, nd)]
        assert np.array_equal(got[1], want[1]), f"replay {r}: routed ids differ"
        assert bits_equal_nan_class(got[2], want[2]), f"replay {r}: routing weights differ"
        assert int(got[3][0]) == int(want[3][0])
        assert bits_equal_nan_class(got[0], want[0]), \
            f"replay {r}: max |diff| {np.abs(got[0] - want[0]).max()}"
    fdm.sync(s.cuda_stream)


def test_noalloc_matches_batched(fdm, layer):
    L = layer
    cases = [(fdm.NOALLOC_MAX_T, 31), (5, 37)]  # the largest step, then a smaller one
    inputs = [tokens(T, seed) for T, seed in cases]
    got = []
    for (T, _), (X, H) in zip(cases, inputs):
        say(f"moe_forward_batched_noalloc L={L} T={T} K={K}")
        got.append(step(fdm, fdm.moe_forward_batched_noalloc, L, X, H, T))
    fdm.sync()
    got = [[to_host(t) for t in g] for g in got]
    for (T, _), (X, H), g in zip(cases, inputs, got):
        say(f"moe_forward_batched L={L} T={T} K={K}")
        want = [to_host(t) for t in step(fdm, fdm.moe_forward_batched, L, X, H, T)]
        fdm.sync()
        assert np.array_equal(g[1], want[1]), f"T={T}: routed ids differ"
        assert bits_equal_nan_class(g[2], want[2]), f"T={T}: routing weights differ"
        assert int(g[3][0]) == int(want[3][0]) == len(np.unique(want[1]))
        assert np.isfinite(want[0]).all()
        assert bits_equal_nan_class(g[0], want[0]), \
            f"T={T}: max |diff| {np.abs(g[0] - want[0]).max()}"


def test_noalloc_rejects_sizes_past_the_scratch(fdm, layer):
    from flash_deepseek_amd._lib import FDM_E_INVAL, FdmError
    L = layer
    T = fdm.NOALLOC_MAX_T + 1
    X, H = tokens(T, 41)
    out = empty_f32(T * 7168)
    with pytest.raises(FdmError) as e:
        fdm.moe_forward_batched_noalloc(L, X, H, T, K, out)
    assert e.value.code == FDM_E_INVAL
    # T within the limit but T*K past FDM_NOALLOC_MAX_PAIRS
    with pytest.raises(FdmError) as e:
        fdm.moe_forward_batched_noalloc(L, X, H, fdm.NOALLOC_MAX_T, 16, out)
    assert e.value.code == FDM_E_INVAL
