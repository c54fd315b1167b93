"""Streamed layers (fdm_layer_stream_open / fdm_moe_layer_streamed): the
reference's expert streaming (infer.m:1478-1602: route, parallel pread of
the selected experts from the packed layer file, experts).  The packed
layer files of the ingest test (sparse, 16 experts with data, Q4_K and Q6_K
down) are streamed through an HBM cache of 8 slots (evictions every token)
and of 256 (everything stays): routing must equal the resident layer's bit
for bit, outputs must agree with it within 1e-4 and with the float64 oracle
within 1e-3, and the cache counters must add up."""
import numpy as np
import pytest

from tests._helpers import empty_f32, rel_l2, say, to_dev, to_host
from tests.test_gpu_ingest import E, H, POP, attach_reference, model, run  # noqa: F401  (model: fixture)

pytestmark = pytest.mark.gpu
K = 8


def run_streamed(fdm, L, h, h_in):
    import torch
    out = empty_f32(H)
    idx = torch.empty(K, dtype=torch.int32, device="cuda")
    w = empty_f32(K)
    fdm.moe_layer_streamed(L, to_dev(h), to_dev(h_in), K, out, idx, w)
    return to_host(out), to_host(idx), to_host(w)


@pytest.mark.parametrize("n_cache", [8, 256])
def test_streamed_matches_resident(fdm, oracle, model, n_cache):
    keep = attach_reference(fdm, model, 50, True)
    _, Wg, bias, shared = keep
    toks = [(oracle.synth_normal(H, 0.0, 1.0, 1200 + t), oracle.synth_normal(H, 0.0, 1.0, 1300 + t))
            for t in range(4)]
    es = model["es"]
    try:
        refs = [run(fdm, 50, h, h_in) for h, h_in in toks]
        say(f"stream_layer q6={model['q6']} n_cache={n_cache}")
        fdm.stream_layer(51, model["packed"], es, Wg, bias, shared, n_cache=n_cache, n_threads=4)
        seen = set()
        for t, ((h, h_in), ref) in enumerate(zip(toks, refs)):
            h0, m0, b0 = fdm.stream_stats(51)
            got = run_streamed(fdm, 51, h, h_in)
            h1, m1, b1 = fdm.stream_stats(51)
            assert np.array_equal(got[1], ref[1]), t
            assert np.array_equal(got[2].view(np.uint32), ref[2].view(np.uint32)), t
            err = rel_l2(got[0], ref[0].astype(np.float64))
            print(f"token {t}: ids {got[1].tolist()} misses {m1 - m0} rel_l2 vs resident {err:.2e}")
            assert err <= 1e-4, t
            ids = set(got[1].tolist())
            assert (h1 - h0) + (m1 - m0) == len(ids)
            if n_cache == 256:
                assert m1 - m0 == len(ids - seen)  # nothing is evicted
            assert b1 - b0 == (m1 - m0) * es
            seen |= ids
        # the first token again: with every expert kept, all hits
        h0, m0, _ = fdm.stream_stats(51)
        again = run_streamed(fdm, 51, *toks[0])
        assert np.array_equal(again[0].view(np.uint32), run_streamed(fdm, 51, *toks[0])[0].view(np.uint32))
        if n_cache == 256:
            assert fdm.stream_stats(51)[1] == m0
        # against the float64 truth on the first token
        h, h_in = toks[0]
        blobs = {e: np.concatenate(model["blobs"][e]) for e in POP}
        want = h_in.astype(np.float64) + oracle.expert_ffn(np.concatenate(model["shared"]), model["q6"], h)
        for e, wk in zip(again[1].tolist(), again[2].tolist()):
            want = want + np.float64(wk) * oracle.expert_ffn(blobs[e], model["q6"], h)
        assert rel_l2(again[0], want) <= 1e-3
    finally:
        fdm.release_layer(51)
        fdm.release_layer(50)
        del keep


def test_stream_errors(fdm, model, tmp_path):
    keep = attach_reference(fdm, model, 50, False)
    _, Wg, bias, _ = keep
    es = model["es"]
    try:
        with pytest.raises(fdm.FdmError):
            fdm.stream_layer(52, tmp_path / "missing.bin", es, Wg, bias)
        short = tmp_path / "short.bin"
        short.write_bytes(b"\0" * 4096)
        with pytest.raises(fdm.FdmError):
            fdm.stream_layer(52, short, es, Wg, bias)
        with pytest.raises(fdm.FdmError):
            fdm.stream_layer(52, model["packed"], es + 1, Wg, bias)
        fdm.stream_layer(52, model["packed"], es, Wg, bias, n_cache=4)
        x = empty_f32(H)
        with pytest.raises(fdm.FdmError):
            fdm.moe_layer_streamed(52, x, None, 8, empty_f32(H))  # K above the cache
        with pytest.raises(fdm.FdmError):
            fdm.moe_layer_streamed(53, x, None, 4, empty_f32(H))  # not streamed
        fdm.release_layer(52)
        with pytest.raises(fdm.FdmError):
            fdm.stream_stats(52)
    finally:
        fdm.release_layer(52)
        fdm.release_layer(50)
        del keep
