"""Helpers shared by the GPU parity tests: moving residues between numpy
(oracle side) and torch device tensors (product side)."""
import numpy as np


def to_dev(a: np.ndarray, dev):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint64)).to(dev)


def to_host(t) -> np.ndarray:
    import torch

    torch.cuda.synchronize(t.device)
    return t.cpu().numpy()


def empty(shape, dev):
    import torch

    return torch.empty(tuple(shape), dtype=torch.uint64, device=dev)


def uniform_limbs(rng: np.random.Generator, shape_prefix, moduli):
    """uint64 residues uniform in [0, q_l) for limb axis -2, shape prefix + (L, N)."""
    *pre, L, N = shape_prefix
    out = np.empty(tuple(pre) + (L, N), dtype=np.uint64)
    for l in range(L):
        out[..., l, :] = rng.integers(0, moduli[l], size=tuple(pre) + (N,), dtype=np.uint64)
    return out


def first_mismatch(a: np.ndarray, b: np.ndarray) -> str:
    if a.shape != b.shape:
        return f"shape {a.shape} != {b.shape}"
    idx = np.argwhere(a != b)
    if len(idx) == 0:
        return "equal"
    i = tuple(idx[0])
    return f"{len(idx)} mismatches, first at {i}: got {a[i]} want {b[i]}"
