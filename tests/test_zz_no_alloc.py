"""pfa_rescale_noalloc, the allocation-free rescale (no reference counterpart):
called through the C ABI it returns exactly pfa_rescale's residues, on two
calls in a row on one context (the second smaller, so a stale scratch would
show), allocates no device memory, and refuses inputs beyond its scratch and
overlapping buffers."""
import numpy as np
import pytest

import py_oracle as O
from gpu_util import empty, first_mismatch, to_dev, to_host, uniform_limbs

pytestmark = pytest.mark.gpu


def test_rescale_noalloc_matches_rescale(dev):
    import torch

    import pfa_native as P

    N = 1 << 16
    mods = O.create_coeff_modulus(N, [60] + [50] * 7 + [60] * 2)
    ctx = P.NativeContext(N, mods, 2)
    rng = np.random.default_rng(77)
    # the allocation-free calls run first, on a stream of their own that no
    # other call has used, so no workspace exists for them to reuse: a call
    # that allocated would show in the device's free memory
    fresh = torch.cuda.Stream(device=dev)
    # two calls in a row: 3 polys at chain 1 (8 limbs), then 2 polys at chain 4
    # (5 limbs) on the same context and stream
    for size, chain in [(3, 1), (2, 4)]:
        L = len(mods) - 2 - (chain - 1)
        x = to_dev(uniform_limbs(rng, (size, L, N), mods[:L]), dev)
        got = empty((size, L - 1, N), dev)
        torch.cuda.synchronize()
        free1 = torch.cuda.mem_get_info()[0]
        ctx.rescale_noalloc(chain, x, got, stream=fresh.cuda_stream)
        ctx.synchronize(fresh.cuda_stream)
        free2 = torch.cuda.mem_get_info()[0]
        # the call itself takes no device memory (a workspace chunk is >= 256 MiB)
        assert free1 - free2 < (16 << 20), (size, chain, free1, free2)
        want = empty((size, L - 1, N), dev)
        ctx.rescale(chain, x, want)
        g, w = to_host(got), to_host(want)
        assert np.array_equal(g, w), (size, chain, first_mismatch(g, w))
    # and against the oracle, so both are pinned
    orc = O.Oracle(N, mods, 2)
    xs = uniform_limbs(rng, (2, 8, N), mods[:8])
    got = empty((2, 7, N), dev)
    ctx.rescale_noalloc(1, to_dev(xs, dev), got)
    g, w = to_host(got), orc.rescale(1, xs, threads=8)
    assert np.array_equal(g, w), first_mismatch(g, w)


def test_rescale_noalloc_errors(dev):
    import pfa_native as P

    N = 1 << 16
    mods = O.create_coeff_modulus(N, [60] + [50] * 3 + [60])
    ctx = P.NativeContext(N, mods, 1)
    x = empty((9, 4, N), dev)  # 9 polys x 2^16 residues: beyond the 2^19-residue scratch
    with pytest.raises(ValueError, match="exceeds its scratch"):
        ctx.rescale_noalloc(1, x, empty((9, 3, N), dev))
    y = empty((2, 4, N), dev)
    with pytest.raises(ValueError, match="overlap"):
        ctx.rescale_noalloc(1, y, y[1:])  # output starts inside the input
    with pytest.raises(ValueError):
        ctx.rescale_noalloc(4, empty((2, 1, N), dev), empty((2, 1, N), dev))  # last level
