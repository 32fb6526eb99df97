"""Loads the committed golden vectors (tests/golden/golden_n1024.npz, written
by tests/golden/make_golden.py from the definitions in plain Python integers)."""
import functools
import os

import numpy as np

PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden_n1024.npz")
N = 1024


@functools.lru_cache(maxsize=1)
def golden():
    with np.load(PATH, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def ints(a):
    return [int(x) for x in a]
