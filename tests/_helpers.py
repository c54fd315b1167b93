"""Helpers shared by the GPU tests (host <-> device copies, error norms)."""
import numpy as np


def to_dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def to_host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def empty_f32(n):
    import torch
    return torch.empty(n, dtype=torch.float32, device="cuda")


def rel_l2(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    den = np.linalg.norm(want)
    return float(np.linalg.norm(got - want) / (den if den > 0 else 1.0))


def bits_equal_nan_class(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    na, nb = np.isnan(a), np.isnan(b)
    return np.array_equal(na, nb) and np.array_equal(a.view(np.uint32)[~na],
                                                     b.view(np.uint32)[~nb])


def say(msg):
    """Name the case before each GPU step (flushed), so a fault names it."""
    print(msg, flush=True)
