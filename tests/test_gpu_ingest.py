"""Real-weight ingest onto the device: a full R1-shape layer written as a
GGUF (stacked expert tensors, router, bias, shared expert; sparse files so
only 16 experts carry data) and as a packed layer file in repack_experts.c's
layout, loaded by fdm_layer_load_gguf / fdm_layer_load_packed.  The loaded
layers must behave bit for bit like the same bytes attached directly
(routing and outputs of fdm_moe_layer), match the oracle run on the bytes
written to the files (routing bit for bit, outputs within 1e-3 relative L2
of float64), and the loaders must reject the
inconsistencies load_layer_weights and repack_experts.c reject."""
import time

import numpy as np
import pytest

from tests import gguf_writer as W
from tests._helpers import empty_f32, rel_l2, say, to_dev, to_host

pytestmark = pytest.mark.gpu

H, F, E = 7168, 2048, 256
GATE = 57344 * 144
POP = sorted(32 * g + o for g in range(8) for o in (5, 21))  # 2 per group of 32


def q4k_blocks(rng, n):
    b = rng.integers(0, 256, (n, 144), dtype=np.uint8)
    d = np.abs(rng.normal(0, 0.02, (n, 2))).astype(np.float16)
    b[:, 0:4] = d.view(np.uint8).reshape(n, 4)
    return b.reshape(-1)


def q6k_blocks(rng, n):
    b = rng.integers(0, 256, (n, 210), dtype=np.uint8)
    d = np.abs(rng.normal(0, 0.02, n)).astype(np.float16)
    b[:, 208:210] = d.view(np.uint8).reshape(n, 2)
    return b.reshape(-1)


def down_blocks(rng, q6):
    return q6k_blocks(rng, 57344) if q6 else q4k_blocks(rng, 57344)


@pytest.fixture(scope="module", params=[False, True], ids=["q4k_down", "q6k_down"])
def model(request, tmp_path_factory):
    """Files on disk + the expected bytes."""
    q6 = request.param
    L = 9
    d = tmp_path_factory.mktemp("model")
    rng = np.random.default_rng(77 + q6)
    down_bytes = 57344 * (210 if q6 else 144)
    es = 2 * GATE + down_bytes
    blobs = {e: (q4k_blocks(rng, 57344), q4k_blocks(rng, 57344), down_blocks(rng, q6)) for e in POP}
    router = rng.normal(0, 0.01, (E, H)).astype(np.float16)
    bias = np.full(E, -5.0, np.float32)
    bias[POP] = rng.normal(0, 0.1, len(POP)).astype(np.float32)
    shared = (q4k_blocks(rng, 57344), q4k_blocks(rng, 57344), down_blocks(rng, q6))
    dt = W.Q6_K if q6 else W.Q4_K
    say(f"writing model files q6={q6}")
    s0 = d / "m-00001-of-00002.gguf"
    s1 = d / "m-00002-of-00002.gguf"
    W.write_gguf(s0, [("general.architecture", W.STRING, "deepseek2")], [
        (f"blk.{L}.ffn_gate_inp.weight", W.F16, (H, E), router.tobytes()),
        (f"blk.{L}.exp_probs_b.bias", W.F32, (E,), bias.tobytes()),
        (f"blk.{L}.ffn_gate_shexp.weight", W.Q4_K, (H, F), shared[0].tobytes()),
        (f"blk.{L}.ffn_up_shexp.weight", W.Q4_K, (H, F), shared[1].tobytes()),
        (f"blk.{L}.ffn_down_shexp.weight", dt, (F, H), shared[2].tobytes())])
    where = W.write_gguf(s1, [], [
        (f"blk.{L}.ffn_gate_exps.weight", W.Q4_K, (H, F, E), None),
        (f"blk.{L}.ffn_up_exps.weight", W.Q4_K, (H, F, E), None),
        (f"blk.{L}.ffn_down_exps.weight", dt, (F, H, E), None)])
    for i, name in enumerate(["gate", "up", "down"]):
        off, _ = where[f"blk.{L}.ffn_{name}_exps.weight"]
        sz = down_bytes if i == 2 else GATE
        W.write_slices(s1, off, [(e * sz, blobs[e][i].tobytes()) for e in POP])
    packed = d / f"layer_{L:02d}.bin"
    with open(packed, "wb") as f:
        f.truncate(E * es)
    W.write_slices(packed, 0, [(e * es, b"".join(x.tobytes() for x in blobs[e])) for e in POP])
    return dict(q6=q6, L=L, es=es, blobs=blobs, router=router, bias=bias, shared=shared,
                shards=[s0, s1], packed=packed)


def attach_reference(fdm, m, L, with_shared=True):
    import torch
    ex = torch.zeros(E * m["es"], dtype=torch.uint8, device="cuda")
    for e, parts in m["blobs"].items():
        ex[e * m["es"]:(e + 1) * m["es"]] = to_dev(np.concatenate(parts))
    wg = to_dev(m["router"].astype(np.float32))
    b = to_dev(m["bias"])
    sh = to_dev(np.concatenate(m["shared"])) if with_shared else None
    fdm.attach_layer(L, ex, m["es"], wg, b, sh)
    return ex, wg, b, sh


def check_oracle(oracle, m, with_shared, h, h_in, got, K=8):
    """A loaded layer against the oracle on the bytes written to the files:
    the routing of the file's router and bias bit for bit, and the output
    within 1e-3 relative L2 of the float64 sum h_in + sum_k w_k E_k (+ S)."""
    out, gi, gw = got
    ri, rw = oracle.route(oracle.router_logits(m["router"].astype(np.float32), h), m["bias"], K=K)
    assert np.array_equal(gi, ri)
    assert np.array_equal(gw.view(np.uint32), rw.view(np.uint32))
    want = h_in.astype(np.float64)
    for e, wk in zip(ri.tolist(), rw.tolist()):
        want = want + np.float64(wk) * oracle.expert_ffn(np.concatenate(m["blobs"][e]), m["q6"], h)
    if with_shared:
        want = want + oracle.expert_ffn(np.concatenate(m["shared"]), m["q6"], h)
    assert rel_l2(out, want) <= 1e-3


def run(fdm, L, h, h_in, K=8):
    import torch
    out = empty_f32(H)
    idx = torch.empty(K, dtype=torch.int32, device="cuda")
    w = empty_f32(K)
    fdm.moe_layer(L, to_dev(h), to_dev(h_in), K, out, idx, w)
    return to_host(out), to_host(idx), to_host(w)


@pytest.mark.parametrize("with_shared", [True, False])
def test_load_gguf_and_packed_match_attached(fdm, oracle, model, with_shared):
    from flash_deepseek_amd import gguf
    L = model["L"]
    keep = attach_reference(fdm, model, 50, with_shared)
    toks = [(oracle.synth_normal(H, 0.0, 1.0, 900 + t), oracle.synth_normal(H, 0.0, 1.0, 950 + t))
            for t in range(3)]
    try:
        refs = [run(fdm, 50, h, h_in) for h, h_in in toks]
        for r in refs:
            assert set(r[1].tolist()) <= set(POP)
        nb = E * model["es"] + (model["es"] if with_shared else 0) + E * H * 4
        with gguf.GGUF(model["shards"]) as m:
            for how in ("gguf", "packed"):
                say(f"load_layer_{how} q6={model['q6']} shared={with_shared}")
                t0 = time.perf_counter()
                if how == "gguf":
                    q6 = gguf.load_layer_gguf(L, m, with_shared)
                else:
                    q6 = gguf.load_layer_packed(L, model["packed"], m, with_shared)
                dt = time.perf_counter() - t0
                print(f"{how} ingest of {nb / 1e9:.2f} GB (sparse files): {nb / dt / 1e9:.2f} GB/s")
                assert q6 == model["q6"]
                assert fdm.layer_info(L) == (model["es"], model["q6"], E)
                for t, ((h, h_in), ref) in enumerate(zip(toks, refs)):
                    got = run(fdm, L, h, h_in)
                    assert np.array_equal(got[1], ref[1])
                    assert np.array_equal(got[2].view(np.uint32), ref[2].view(np.uint32))
                    assert np.array_equal(got[0].view(np.uint32), ref[0].view(np.uint32))
                    if t == 0:
                        check_oracle(oracle, model, with_shared, h, h_in, got)
                fdm.release_layer(L)
    finally:
        fdm.release_layer(50)
        del keep


def test_load_rejects(fdm, model, tmp_path):
    from flash_deepseek_amd import gguf
    from flash_deepseek_amd._lib import FDM_E_FORMAT, FDM_E_SIZE, FdmError
    with gguf.GGUF(model["shards"]) as m:
        with pytest.raises(FdmError) as e:          # no such layer in the file
            gguf.load_layer_gguf(model["L"] + 3, m)
        assert e.value.code == FDM_E_FORMAT
        bad = tmp_path / "short.bin"
        with open(bad, "wb") as f:
            f.truncate(E * model["es"] - E)          # not two Q4_K + a known down
        with pytest.raises(FdmError) as e:
            gguf.load_layer_packed(model["L"], bad, m)
        assert e.value.code == FDM_E_SIZE
    # shared down type differing from the routed experts'
    L = 4
    p = tmp_path / "mixed.gguf"
    dt, st = (W.Q4_K, W.Q6_K) if not model["q6"] else (W.Q6_K, W.Q4_K)
    W.write_gguf(p, [], [
        (f"blk.{L}.ffn_gate_exps.weight", W.Q4_K, (H, F, E), None),
        (f"blk.{L}.ffn_up_exps.weight", W.Q4_K, (H, F, E), None),
        (f"blk.{L}.ffn_down_exps.weight", dt, (F, H, E), None),
        (f"blk.{L}.ffn_gate_inp.weight", W.F32, (H, E), None),
        (f"blk.{L}.ffn_gate_shexp.weight", W.Q4_K, (H, F), None),
        (f"blk.{L}.ffn_up_shexp.weight", W.Q4_K, (H, F), None),
        (f"blk.{L}.ffn_down_shexp.weight", st, (F, H), None)])
    with gguf.GGUF(p) as m:
        with pytest.raises(FdmError) as e:
            gguf.load_layer_gguf(L, m, with_shared=True)
        assert e.value.code == FDM_E_FORMAT
        # without the shared expert the same file loads (router F32, no bias)
        assert gguf.load_layer_gguf(L, m, with_shared=False) == (dt == W.Q6_K)
        fdm.release_layer(L)
