"""Seeded synthetic MoE layers of DeepSeek-R1 shape, generated on the device
by the library's own generator (fdm_synth_*).  Used by the benchmark and the
parity tests: there are no real weights in this environment.

Workload (per layer):
  routed experts  256 packed blobs [gate Q4_K 2048x7168 | up Q4_K | down
                  Q4_K or Q6_K 7168x2048]; Q4_K d, dmin = fp16(|N(0,0.02)|),
                  scale and qs bytes uniform; Q6_K ql/qh uniform, int8 scales
                  uniform on -128..127, d = fp16(|N(0,0.02)|)
  shared expert   one more blob of the same layout
  router          W_g fp32 N(0, 0.01) [256 x 7168], bias fp32 N(0, 0.1)
"""
from dataclasses import dataclass

from . import (EXPERT_Q4K_BYTES, EXPERT_Q6K_BYTES, HIDDEN, N_EXPERTS, synth_normal, synth_q4k,
               synth_q6k)

GATE_BYTES = 57344 * 144
MASK64 = (1 << 64) - 1


def blob_seed(layer_seed, expert, matrix):
    """Seed of matrix `matrix` (0 gate, 1 up, 2 down) of expert `expert`
    (-1 = shared) of the layer with seed `layer_seed`."""
    return (layer_seed * 0x100000001B3 + (expert + 1) * 8 + matrix + 1) & MASK64


@dataclass
class SynthLayer:
    experts: object  # uint8 tensor, n_experts * expert_size
    shared: object   # uint8 tensor, expert_size
    Wg: object       # float32 [256, 7168]
    bias: object     # float32 [256]
    expert_size: int
    down_q6: bool

    def expert_bytes(self, e):
        """Host copy of expert e's packed blob (e = -1: the shared expert)."""
        import torch
        torch.cuda.synchronize()
        if e < 0:
            return self.shared.cpu().numpy()
        s = self.expert_size
        return self.experts[e * s:(e + 1) * s].cpu().numpy()


def fill_blob(dst, base, layer_seed, expert, down_q6):
    """Write one packed expert into the uint8 tensor `dst` at byte `base`."""
    p = dst.data_ptr() + base
    synth_q4k(p, 57344, blob_seed(layer_seed, expert, 0))
    synth_q4k(p + GATE_BYTES, 57344, blob_seed(layer_seed, expert, 1))
    if down_q6:
        synth_q6k(p + 2 * GATE_BYTES, 57344, blob_seed(layer_seed, expert, 2))
    else:
        synth_q4k(p + 2 * GATE_BYTES, 57344, blob_seed(layer_seed, expert, 2))


def make_layer(layer_seed, down_q6=False, n_experts=N_EXPERTS):
    import torch
    size = EXPERT_Q6K_BYTES if down_q6 else EXPERT_Q4K_BYTES
    experts = torch.empty(n_experts * size, dtype=torch.uint8, device="cuda")
    shared = torch.empty(size, dtype=torch.uint8, device="cuda")
    for e in range(n_experts):
        fill_blob(experts, e * size, layer_seed, e, down_q6)
    fill_blob(shared, 0, layer_seed, -1, down_q6)
    Wg = torch.empty((N_EXPERTS, HIDDEN), dtype=torch.float32, device="cuda")
    bias = torch.empty(N_EXPERTS, dtype=torch.float32, device="cuda")
    synth_normal(Wg, Wg.numel(), 0.0, 0.01, (layer_seed * 31 + 7) & MASK64)
    synth_normal(bias, N_EXPERTS, 0.0, 0.1, (layer_seed * 31 + 8) & MASK64)
    return SynthLayer(experts, shared, Wg, bias, size, down_q6)


def make_tokens(n, seed, mean=0.0, std=1.0):
    """n x 7168 fp32 activations N(mean, std) on the device."""
    import torch
    x = torch.empty((n, HIDDEN), dtype=torch.float32, device="cuda")
    synth_normal(x, x.numel(), mean, std, seed & MASK64)
    return x
