"""Concurrent calls from several host threads, each on its own stream.

Every call that needs scratch memory takes it from its stream's workspace,
so threads on different streams may overlap.  Two threads, each on its own
torch stream, loop over the batch-1 layer, the batched step (grouped MFMA
GEMMs) and prefill on their own inputs; every result must carry the same
bits as the same call made alone on the null stream beforehand.  Then one
stream's workspace is released and made again by its next call."""
import threading

import numpy as np
import pytest

from tests._helpers import empty_f32, say, to_dev, to_host

pytestmark = pytest.mark.gpu

L = 14
K = 8
T_BATCH = 32
T_PREFILL = 48
ROUNDS = 12


@pytest.fixture(scope="module")
def layer(fdm):
    from flash_deepseek_amd.synthetic import make_layer
    say(f"building layer L={L}")
    lay = make_layer(3000 + L)
    fdm.attach_layer(L, lay.experts, lay.expert_size, lay.Wg, lay.bias, lay.shared)
    yield lay
    fdm.release_layer(L)


def inputs(oracle, seed):
    h = oracle.synth_normal(7168, 0.0, 1.0, seed)
    h_in = oracle.synth_normal(7168, 0.0, 1.0, seed + 1)
    X = np.stack([oracle.synth_normal(7168, 0.0, 1.0, seed + 10 + t) for t in range(T_BATCH)])
    H = np.stack([oracle.synth_normal(7168, 0.0, 1.0, seed + 100 + t) for t in range(T_PREFILL)])
    nw = oracle.synth_normal(7168, 1.0, 0.1, seed + 500)
    return {k: to_dev(v.ravel()) for k, v in dict(h=h, h_in=h_in, X=X, H=H, nw=nw).items()}


def run_all(fdm, x, stream):
    """The three calls on `stream` (None: the null stream); device outputs."""
    import torch
    dev = torch.device("cuda")
    with torch.cuda.stream(stream if stream is not None else torch.cuda.default_stream(dev)):
        s = stream.cuda_stream if stream is not None else 0
        hid = empty_f32(7168)
        fdm.moe_layer(L, x["h"], x["h_in"], K, hid, stream=s)
        out = empty_f32(T_BATCH * 7168)
        fdm.moe_forward_batched(L, x["X"], x["X"], T_BATCH, K, out, stream=s)
        H = x["H"].clone()
        fdm.moe_prefill([L], H, T_PREFILL, K, [x["nw"]], stream=s)
    return hid, out, H


def bits(ts):
    return [to_host(t).view(np.uint32) for t in ts]


def test_two_threads_two_streams(fdm, oracle, layer):
    import torch
    xs = [inputs(oracle, 41000), inputs(oracle, 42000)]
    say("reference calls on the null stream")
    want = [bits(run_all(fdm, x, None)) for x in xs]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    got = [[], []]
    errors = []

    def worker(i):
        try:
            for _ in range(ROUNDS):
                got[i].append(run_all(fdm, xs[i], streams[i]))
            fdm.sync(streams[i].cuda_stream)
        except Exception as e:  # reported below, from the main thread
            errors.append(e)

    say(f"two threads x {ROUNDS} rounds of moe_layer / moe_forward_batched T={T_BATCH} / prefill T={T_PREFILL}")
    th = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for t in th:
        t.start()
    for t in th:
        t.join(timeout=100)
    assert not any(t.is_alive() for t in th), "a worker thread did not finish"
    assert not errors, errors
    torch.cuda.synchronize()
    for i in range(2):
        assert len(got[i]) == ROUNDS
        for r, res in enumerate(got[i]):
            for name, a, b in zip(("moe_layer", "batched", "prefill"), bits(res), want[i]):
                assert np.array_equal(a, b), f"thread {i} round {r}: {name} differs from the null-stream call"

    say("stream_release, then the stream's next call makes a new workspace")
    fdm.stream_release(streams[0])
    again = bits(run_all(fdm, xs[0], streams[0]))
    fdm.sync(streams[0].cuda_stream)
    for a, b in zip(again, want[0]):
        assert np.array_equal(a, b)
    for s in streams:
        fdm.stream_release(s)
