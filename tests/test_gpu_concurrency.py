"""Several host threads, each with its own stream, calling the fused
key-switching entry points on one context at once, as a serving process does.
The workspace is per (thread, stream) and the lazily built work tables take a
lock.  Each result must equal the same call run alone, and no device error
(e.g. a split inner-product item whose chunks ran on two XCDs) may be
recorded."""
import threading

import numpy as np
import pytest

from gpu_util import empty, first_mismatch, to_dev, to_host, uniform_limbs
from test_gpu_keyswitch import Setup

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("logN,nq,alpha", [(16, 24, 4), (13, 8, 2)])
def test_streams_concurrent_keyswitch(dev, logN, nq, alpha):
    """Config 3's shape (whose inner product splits its left-over items into
    digit chunks) and a small one: three threads, each on its own stream, each
    enqueueing 6 fused HMult + relinearize + rescale calls, 6 rotations and 6
    pairs of hoisted rotations, concurrently."""
    import torch

    import pfa_native as P

    st = Setup(logN, nq, alpha, seed=99 + logN)
    N, chain = st.N, 1
    Ql = st.orc.size_Ql(chain)
    key = to_dev(uniform_limbs(st.rng, (st.orc.dnum, 2, st.QP, N), st.mods), dev)
    T, REPS = 3, 6
    a = [to_dev(st.ct(chain), dev) for _ in range(T)]
    b = [to_dev(st.ct(chain), dev) for _ in range(T)]
    elts = [P.galois_elt_from_step(s, N) for s in (1, -7, 33)]
    want_m, want_r, want_h = [], [], []
    for i in range(T):
        o = empty((2, Ql - 1, N), dev)
        st.ctx.multiply_relin_rescale(chain, a[i], b[i], key, o)
        want_m.append(to_host(o))
        d = a[i].clone()
        st.ctx.apply_galois(chain, d, elts[i], key)
        want_r.append(to_host(d))
        h = empty((2, 2, Ql, N), dev)
        st.ctx.hoist_rotations(chain, b[i], elts[:2], [key, key], h)
        want_h.append(to_host(h))
    torch.cuda.synchronize()
    results, errors = [None] * T, []

    def work(i):
        try:
            s = torch.cuda.Stream()
            outs = []
            with torch.cuda.stream(s):
                for _ in range(REPS):
                    o = empty((2, Ql - 1, N), dev)
                    st.ctx.multiply_relin_rescale(chain, a[i], b[i], key, o)
                    d = a[i].clone()
                    st.ctx.apply_galois(chain, d, elts[i], key)
                    h = empty((2, 2, Ql, N), dev)
                    st.ctx.hoist_rotations(chain, b[i], elts[:2], [key, key], h)
                    outs.append((o, d, h))
            st.ctx.synchronize(s.cuda_stream)
            results[i] = [(o.cpu().numpy(), d.cpu().numpy(), h.cpu().numpy()) for o, d, h in outs]
        except Exception as e:  # reported below
            errors.append((i, repr(e)))

    threads = [threading.Thread(target=work, args=(i,)) for i in range(T)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert errors == []
    for i in range(T):
        for rep, (m, r, h) in enumerate(results[i]):
            assert np.array_equal(m, want_m[i]), ("hmult", i, rep, first_mismatch(m, want_m[i]))
            assert np.array_equal(r, want_r[i]), ("rotate", i, rep, first_mismatch(r, want_r[i]))
            assert np.array_equal(h, want_h[i]), ("hoist", i, rep, first_mismatch(h, want_h[i]))
