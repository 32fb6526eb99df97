"""A seeded random sweep of key-switching shapes, each checked bit for bit
against the oracle: chains of 2-12 primes drawn from 30 to 60 bits (so both
arithmetic policies mix within a chain, in any order), alpha 1-4 special
primes of random sizes, any level the key covers, N = 2^12 and 2^13.

Per shape: the fused multiply + relinearize + rescale (src/evaluate.cu:
1061-1104, src/rns.cu:1128-1184) alone and as a batch of two, a rotation
(src/evaluate.cu:1607-1656) alone and as a batch of two with different steps
and keys, and hoisted rotations (src/evaluate.cu:1929-2082).  The fixed shapes
of test_gpu_keyswitch.py pin the regular cases; this sweep covers prime-size
orders and digit splits no hand-picked list does.  Two further tests take the
limits: digits of 5 to 16 special primes, and 20 hoisted rotations / a batch
of 70 rotations (past the per-launch groups and work-schedule sizes).
"""
import numpy as np
import pytest

import py_oracle as O
from gpu_util import empty, first_mismatch, to_dev, to_host, uniform_limbs
from test_gpu_keyswitch import Setup

pytestmark = pytest.mark.gpu

SIZES = [30, 36, 40, 45, 49, 50, 55, 58, 60]


def _shapes(n, seed):
    """(logN, nq, alpha, chain, bits) with the key covering the level
    (beta(chain) <= dnum = nq // alpha, the reference's digit count)."""
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        logN = int(rng.choice([12, 13]))
        nq = int(rng.integers(2, 13))
        alpha = int(rng.integers(1, 5))
        if nq // alpha < 1:
            continue
        chain = int(rng.integers(1, nq))  # at least 2 primes left, so the rescale has a target
        Ql = nq - chain + 1
        if -(-Ql // alpha) > nq // alpha:
            continue
        bits = [int(b) for b in rng.choice(SIZES, size=nq + alpha)]
        out.append((logN, nq, alpha, chain, bits))
    return out


SHAPES = _shapes(12, 2024)


@pytest.mark.parametrize("logN,nq,alpha,chain,bits", SHAPES)
def test_random_shape_bit_exact(dev, logN, nq, alpha, chain, bits):
    import pfa_native as P

    st = Setup(logN, nq, alpha, seed=sum(bits) + chain, bits=bits)
    orc, N = st.orc, st.N
    assert orc.beta(chain) <= orc.dnum
    Ql = orc.size_Ql(chain)
    keys = [st.key() for _ in range(2)]
    dkeys = [to_dev(k, dev) for k in keys]

    # fused HMult, single and batched
    a = np.stack([st.ct(chain) for _ in range(2)])
    b = np.stack([st.ct(chain) for _ in range(2)])
    want = [orc.rescale(chain, orc.multiply_and_relin(chain, a[i], b[i], keys[0], threads=8), threads=8)
            for i in range(2)]
    one = empty((2, Ql - 1, N), dev)
    st.ctx.multiply_relin_rescale(chain, to_dev(a[0], dev), to_dev(b[0], dev), dkeys[0], one)
    got = to_host(one)
    assert np.array_equal(got, want[0]), ("hmult", first_mismatch(got, want[0]))
    two = empty((2, 2, Ql - 1, N), dev)
    st.ctx.multiply_relin_rescale_batch(chain, 2, to_dev(a, dev), to_dev(b, dev), dkeys[0], two)
    got = to_host(two)
    for i in range(2):
        assert np.array_equal(got[i], want[i]), ("hmult batch", i, first_mismatch(got[i], want[i]))

    # rotations: one, a batch of two (own step and key each), hoisted
    rng = np.random.default_rng(Ql)
    steps = [int(s) for s in rng.integers(-N // 4, N // 4, size=2)]
    elts = [P.galois_elt_from_step(s, N) for s in steps]
    cts = np.stack([st.ct(chain) for _ in range(2)])
    d = to_dev(cts[0], dev)
    st.ctx.apply_galois(chain, d, elts[0], dkeys[0])
    want_rot = [orc.apply_galois(chain, cts[i], elts[i], keys[i], threads=8) for i in range(2)]
    got = to_host(d)
    assert np.array_equal(got, want_rot[0]), ("rotate", first_mismatch(got, want_rot[0]))
    out = empty(cts.shape, dev)
    st.ctx.rotate_batch(chain, to_dev(cts, dev), elts, dkeys, out)
    got = to_host(out)
    for i in range(2):
        assert np.array_equal(got[i], want_rot[i]), ("rotate batch", i, first_mismatch(got[i], want_rot[i]))
    hoisted = empty((2, 2, Ql, N), dev)
    st.ctx.hoist_rotations(chain, to_dev(cts[0], dev), elts, dkeys, hoisted)
    want_h = orc.hoist_rotations(chain, cts[0], elts, keys, threads=8)
    got = to_host(hoisted)
    assert np.array_equal(got, want_h), ("hoist", first_mismatch(got, want_h))
    st.ctx.synchronize()


def test_random_shapes_cover_both_policies():
    """The sweep mixes FP64-policy (< 2^50) and integer-policy primes in its
    chains and special primes, and reaches alpha 1 to 4 and lower levels."""
    assert {s[2] for s in SHAPES} == {1, 2, 3, 4}
    assert any(s[3] > 1 for s in SHAPES)
    assert all(any(b < 50 for b in s[4]) or any(b >= 50 for b in s[4]) for s in SHAPES)
    assert sum(1 for s in SHAPES if any(b < 50 for b in s[4]) and any(b >= 50 for b in s[4])) >= 8


@pytest.mark.parametrize("nq,alpha", [(16, 8), (16, 16), (18, 6)])
def test_wide_digits_bit_exact(dev, nq, alpha):
    """Digits of 5 to 16 special primes (the library's limit is 16): the fused
    HMult + relinearize + rescale, a rotation and hoisted rotations against the
    oracle, with 60-bit and 50-bit primes mixed in the chain and the digits."""
    import pfa_native as P

    bits = [60] + [50, 55, 36, 60] * 8
    st = Setup(12, nq, alpha, seed=nq * alpha, bits=bits[:nq] + ([60, 49] * 8)[:alpha])
    orc, N = st.orc, st.N
    chain = 1
    Ql = orc.size_Ql(chain)
    assert orc.beta(chain) <= orc.dnum
    key = st.key()
    dkey = to_dev(key, dev)
    a, b = st.ct(chain), st.ct(chain)
    want = orc.rescale(chain, orc.multiply_and_relin(chain, a, b, key, threads=8), threads=8)
    out = empty((2, Ql - 1, N), dev)
    st.ctx.multiply_relin_rescale(chain, to_dev(a, dev), to_dev(b, dev), dkey, out)
    got = to_host(out)
    assert np.array_equal(got, want), ("hmult", first_mismatch(got, want))
    elt = P.galois_elt_from_step(-9, N)
    ct = st.ct(chain)
    d = to_dev(ct, dev)
    st.ctx.apply_galois(chain, d, elt, dkey)
    got, want = to_host(d), orc.apply_galois(chain, ct, elt, key, threads=8)
    assert np.array_equal(got, want), ("rotate", first_mismatch(got, want))
    elts = [P.galois_elt_from_step(s, N) for s in (1, 5)]
    hoisted = empty((2, 2, Ql, N), dev)
    st.ctx.hoist_rotations(chain, d, elts, [dkey, dkey], hoisted)
    want = orc.hoist_rotations(chain, to_host(d), elts, [key, key], threads=8)
    got = to_host(hoisted)
    assert np.array_equal(got, want), ("hoist", first_mismatch(got, want))


def test_many_rotations_bit_exact(dev):
    """20 hoisted rotations (two groups of the launcher's 16 per ModDown), their
    sum (hoisting), and a rotation batch of 70 members (past the 64-member work
    schedules), against the oracle's hoist_rotations / hoisting / apply_galois."""
    import pfa_native as P

    st = Setup(12, 4, 2, seed=20, bits=[60, 50, 50, 50, 60, 60])
    orc, N, chain = st.orc, st.N, 1
    Ql = orc.size_Ql(chain)
    keys = [st.key() for _ in range(4)]
    dkeys = [to_dev(k, dev) for k in keys]
    steps = list(range(1, 21))
    elts = [P.galois_elt_from_step(s, N) for s in steps]
    ct = st.ct(chain)
    out = empty((20, 2, Ql, N), dev)
    st.ctx.hoist_rotations(chain, to_dev(ct, dev), elts, [dkeys[i % 4] for i in range(20)], out)
    want = orc.hoist_rotations(chain, ct, elts, [keys[i % 4] for i in range(20)], threads=8)
    got = to_host(out)
    assert np.array_equal(got, want), ("hoist 20", first_mismatch(got, want))
    # the sum of the 20 rotations (hoisting: one launch for all members)
    summed = empty((2, Ql, N), dev)
    st.ctx.hoisting(chain, to_dev(ct, dev), elts, [dkeys[i % 4] for i in range(20)], summed)
    want = orc.hoisting(chain, ct, elts, [keys[i % 4] for i in range(20)], threads=8)
    got = to_host(summed)
    assert np.array_equal(got, want), ("hoisting 20", first_mismatch(got, want))
    cts = np.stack([st.ct(chain) for _ in range(70)])
    belts = [elts[i % 20] for i in range(70)]
    out = empty(cts.shape, dev)
    st.ctx.rotate_batch(chain, to_dev(cts, dev), belts, [dkeys[i % 4] for i in range(70)], out)
    got = to_host(out)
    for i in range(70):
        want = orc.apply_galois(chain, cts[i], belts[i], keys[i % 4], threads=8)
        assert np.array_equal(got[i], want), ("rotate batch", i, first_mismatch(got[i], want))
