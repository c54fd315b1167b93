"""Seeded MLA attention weights of R1 shape for the attention tests, in the
layout LayerAttnDense holds (infer.m:687-706); F16 matrices as uint16
bits, norms float32.  Scales keep every intermediate O(1)."""
import numpy as np

H, NH, QA, KVL, NOPE, ROPE, QK, VH = 7168, 128, 1536, 512, 128, 64, 192, 128


def mla_weights(seed):
    rng = np.random.default_rng(seed)

    def f16(shape, fan_in):
        return (rng.standard_normal(shape, dtype=np.float32) * fan_in ** -0.5).astype(np.float16).view(np.uint16)

    return {
        "attn_norm": rng.normal(1.0, 0.1, H).astype(np.float32),
        "q_a": f16((QA, H), H),
        "q_a_norm": rng.normal(1.0, 0.1, QA).astype(np.float32),
        "q_b": f16((NH * QK, QA), QA),
        "kv_a": f16((KVL + ROPE, H), H),
        "kv_a_norm": rng.normal(1.0, 0.1, KVL).astype(np.float32),
        "k_b": f16((NH, KVL, NOPE), NOPE),
        "v_b": f16((NH, VH, KVL), KVL),
        "o_proj": f16((H, NH * VH), NH * VH),
    }
