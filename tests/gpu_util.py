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


def _is_prime64(n: int) -> bool:
    """Deterministic Miller-Rabin for n < 2^64 (the first 12 prime bases)."""
    if n < 2:
        return False
    small = (2, 3, 5, 7, 11, 13, 17, 19, 23, 29, 31, 37)
    for p in small:
        if n % p == 0:
            return n == p
    d, s = n - 1, 0
    while d % 2 == 0:
        d, s = d // 2, s + 1
    for a in small:
        x = pow(a, d, n)
        if x in (1, n - 1):
            continue
        for _ in range(s - 1):
            x = x * x % n
            if x == n - 1:
                break
        else:
            return False
    return True


def primes_near_2_61(N: int, count: int) -> list:
    """The `count` largest primes q = 1 mod 2N below 2^61 (the context's limit),
    in decreasing order: products of their residues come within a factor of
    2^-6 of 2^122, so 65 of them pass 2^128."""
    out, q = [], ((1 << 61) - 2) // (2 * N) * (2 * N) + 1
    while len(out) < count:
        if _is_prime64(q):
            out.append(q)
        q -= 2 * N
    return out
