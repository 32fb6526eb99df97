"""GPU parity of the key-switching path and the evaluator entry points against
the CPU oracle, bit-exact on every RNS residue:

  tensor (src/polymath.cu:463-498), ModUp (src/rns_bconv.cu:530-628), the
  inner product (src/eval_key_switch.cu:175-230), ModDown
  (src/rns_bconv.cu:776-828), keyswitch_inplace (src/eval_key_switch.cu:294-381),
  multiply_and_relin (src/evaluate.cu:1061-1104), rescale
  (src/rns.cu:1128-1184), the Galois permutation and rotation
  (src/galois.cu, src/evaluate.cu:1607-1656), hoisted rotations
  (src/evaluate.cu:1929-2082) and key construction (src/secretkey.cu:354-398).

Shapes cover alpha = 1 (the single-special-prime BConv), a short last digit
(|Ql| not a multiple of alpha), lower levels (chain index > 1) and the benchmark
config-3 shape (N = 2^16, |Q| = 24, alpha = 4, dnum = 6).
"""
import numpy as np
import pytest

import py_oracle as O
from gpu_util import empty, first_mismatch, to_dev, to_host, uniform_limbs

pytestmark = pytest.mark.gpu

SHAPES = [  # (logN, nq, alpha, chain)
    (12, 6, 2, 1),
    (12, 8, 3, 4),   # short last digit (|Ql| = 5, alpha = 3), lower level
    (12, 5, 1, 2),   # alpha = 1
    (12, 6, 3, 2),   # lower level, short last digit
    (13, 8, 4, 1),
    (16, 6, 2, 3),
]
# ModUp / ModDown need no key, so they also take the top level of a chain whose
# |Q| is not a multiple of alpha (beta = 4 > dnum = 3: keys cannot serve it).
KEYLESS_SHAPES = SHAPES + [(12, 7, 2, 1)]


def chain_bits(nq, alpha):
    return [60] + [50] * (nq - 1) + [60] * alpha


class Setup:
    def __init__(self, logN, nq, alpha, seed=0, bits=None):
        import pfa_native as P

        self.N = 1 << logN
        self.mods = O.create_coeff_modulus(self.N, bits or chain_bits(nq, alpha))
        self.nq, self.alpha = nq, alpha
        self.ctx = P.NativeContext(self.N, self.mods, alpha)
        self.orc = O.Oracle(self.N, self.mods, alpha)
        self.rng = np.random.default_rng(seed)
        self.QP = len(self.mods)

    def qlp_mods(self, chain):
        Ql = self.orc.size_Ql(chain)
        return self.mods[:Ql] + self.mods[self.nq:]

    def ct(self, chain, size=2):
        Ql = self.orc.size_Ql(chain)
        return uniform_limbs(self.rng, (size, Ql, self.N), self.mods[:Ql])

    def key(self):
        """A well-formed key switching key [dnum][2][QP][N] from uniform a and small e (via the oracle)."""
        o, N = self.orc, self.N
        s = np.zeros(N, dtype=np.int64)
        idx = self.rng.choice(N, size=min(64, N), replace=False)
        s[idx] = self.rng.choice([-1, 1], size=len(idx))
        S = o.ntt_fwd(np.stack([(s % q).astype(np.uint64) for q in self.mods]), threads=8)
        new = uniform_limbs(self.rng, (self.QP, N), self.mods)
        a = uniform_limbs(self.rng, (o.dnum, self.QP, N), self.mods)
        e = uniform_limbs(self.rng, (o.dnum, self.QP, N), self.mods)
        return o.kswitch_key(new, S, a, e)


@pytest.mark.parametrize("logN,nq,alpha,chain", KEYLESS_SHAPES)
def test_modup(dev, logN, nq, alpha, chain):
    st = Setup(logN, nq, alpha, seed=1)
    Ql = st.orc.size_Ql(chain)
    c2 = uniform_limbs(st.rng, (Ql, st.N), st.mods)
    out = empty((st.orc.beta(chain), Ql + alpha, st.N), dev)
    st.ctx.modup(chain, to_dev(c2, dev), out)
    got, want = to_host(out), st.orc.modup(chain, c2, threads=8)
    assert np.array_equal(got, want), first_mismatch(got, want)


@pytest.mark.parametrize("logN,nq,alpha,chain", SHAPES)
def test_inner_product(dev, logN, nq, alpha, chain):
    st = Setup(logN, nq, alpha, seed=2)
    Ql = st.orc.size_Ql(chain)
    beta = st.orc.beta(chain)
    t = uniform_limbs(st.rng, (beta, Ql + alpha, st.N), st.qlp_mods(chain))
    key = uniform_limbs(st.rng, (st.orc.dnum, 2, st.QP, st.N), st.mods)
    cx = empty((2, Ql + alpha, st.N), dev)
    st.ctx.ks_inner_prod(chain, to_dev(t, dev), to_dev(key, dev), cx)
    got, want = to_host(cx), st.orc.ks_inner_prod(chain, t, key)
    assert np.array_equal(got, want), first_mismatch(got, want)


def test_inner_product_many_digits(dev):
    """70 one-prime digits below primes near 2^61 at N = 2^10, with maximal
    residues at half the positions: 65 such products pass 2^128, so the staged
    inner product must fold its 128-bit sums on the way (the reference folds at
    a threshold from the prime sizes, src/eval_key_switch.cu:175-230); the fused
    multiply_and_relin (src/evaluate.cu:1061-1104) at the same depth too."""
    import pfa_native as P
    from gpu_util import primes_near_2_61

    N, nq, alpha, chain = 1 << 10, 70, 1, 1
    mods = primes_near_2_61(N, nq + alpha)
    ctx, orc = P.NativeContext(N, mods, alpha), O.Oracle(N, mods, alpha)
    Ql, beta, QP = orc.size_Ql(chain), orc.beta(chain), len(mods)
    assert beta == 70 and beta * (min(mods) - 1) ** 2 >= 1 << 128
    rng = np.random.default_rng(70)
    qlp = np.array(mods[:Ql] + mods[nq:], dtype=np.uint64)
    t = uniform_limbs(rng, (beta, Ql + alpha, N), list(qlp))
    t[..., : N // 2] = (qlp - 1)[None, :, None]
    key = uniform_limbs(rng, (orc.dnum, 2, QP, N), mods)
    key[..., : N // 2] = (np.array(mods, dtype=np.uint64) - 1)[None, None, :, None]
    dkey = to_dev(key, dev)
    cx = empty((2, Ql + alpha, N), dev)
    ctx.ks_inner_prod(chain, to_dev(t, dev), dkey, cx)
    got, want = to_host(cx), orc.ks_inner_prod(chain, t, key)
    assert np.array_equal(got, want), ("inner product", first_mismatch(got, want))
    a = uniform_limbs(rng, (2, Ql, N), mods[:Ql])
    b = uniform_limbs(rng, (2, Ql, N), mods[:Ql])
    out = empty((2, Ql, N), dev)
    ctx.multiply_and_relin(chain, to_dev(a, dev), to_dev(b, dev), dkey, out)
    got, want = to_host(out), orc.multiply_and_relin(chain, a, b, key, threads=8)
    assert np.array_equal(got, want), ("multiply_and_relin", first_mismatch(got, want))


@pytest.mark.parametrize("logN,nq,alpha,chain", KEYLESS_SHAPES)
def test_moddown(dev, logN, nq, alpha, chain):
    st = Setup(logN, nq, alpha, seed=3)
    Ql = st.orc.size_Ql(chain)
    cx = uniform_limbs(st.rng, (Ql + alpha, st.N), st.qlp_mods(chain))
    out = empty((Ql, st.N), dev)
    st.ctx.moddown(chain, to_dev(cx, dev), out)
    got, want = to_host(out), st.orc.moddown(chain, cx, threads=8)
    assert np.array_equal(got, want), first_mismatch(got, want)


@pytest.mark.parametrize("logN,nq,alpha,chain", SHAPES)
def test_keyswitch(dev, logN, nq, alpha, chain):
    st = Setup(logN, nq, alpha, seed=4)
    Ql = st.orc.size_Ql(chain)
    ct = st.ct(chain)
    c2 = uniform_limbs(st.rng, (Ql, st.N), st.mods)
    key = st.key()
    d = to_dev(ct, dev)
    st.ctx.keyswitch(chain, d, to_dev(c2, dev), to_dev(key, dev))
    got, want = to_host(d), st.orc.keyswitch(chain, ct, c2, key, threads=8)
    assert np.array_equal(got, want), first_mismatch(got, want)


@pytest.mark.parametrize("logN,nq,alpha,chain", SHAPES[:3])
def test_tensor_and_relinearize(dev, logN, nq, alpha, chain):
    st = Setup(logN, nq, alpha, seed=5)
    Ql = st.orc.size_Ql(chain)
    a, b = st.ct(chain), st.ct(chain)
    out3 = empty((3, Ql, st.N), dev)
    st.ctx.tensor(chain, to_dev(a, dev), to_dev(b, dev), out3)
    want3 = st.orc.tensor(a, b)
    assert np.array_equal(to_host(out3), want3)
    key = st.key()
    out = empty((2, Ql, st.N), dev)
    st.ctx.relinearize(chain, out3, to_dev(key, dev), out)
    want = st.orc.keyswitch(chain, want3[:2], want3[2], key, threads=8)
    assert np.array_equal(to_host(out), want)


@pytest.mark.parametrize("logN,nq,alpha,chain", SHAPES)
def test_multiply_and_relin(dev, logN, nq, alpha, chain):
    st = Setup(logN, nq, alpha, seed=6)
    Ql = st.orc.size_Ql(chain)
    a, b = st.ct(chain), st.ct(chain)
    key = st.key()
    out = empty((2, Ql, st.N), dev)
    st.ctx.multiply_and_relin(chain, to_dev(a, dev), to_dev(b, dev), to_dev(key, dev), out)
    got, want = to_host(out), st.orc.multiply_and_relin(chain, a, b, key, threads=8)
    assert np.array_equal(got, want), first_mismatch(got, want)


@pytest.mark.parametrize("alias", ["a", "b", "ab"])
def test_multiply_and_relin_in_place(dev, alias):
    """multiply_and_relin in place (out aliasing a, b or both): the tensor
    product is formed before the key switch overwrites out, so the residues
    equal the oracle's."""
    st = Setup(12, 6, 2, seed=8)
    a, b = st.ct(1), st.ct(1)
    key = st.key()
    da = to_dev(a, dev)
    db = da if alias == "ab" else to_dev(b, dev)
    out = db if alias == "b" else da
    st.ctx.multiply_and_relin(1, da, db, to_dev(key, dev), out)
    got, want = to_host(out), st.orc.multiply_and_relin(1, a, a if alias == "ab" else b, key, threads=8)
    assert np.array_equal(got, want), first_mismatch(got, want)


def test_multiply_and_relin_config3(dev):
    """benchmark config 3 shape: N = 2^16, chain {60, 50 x 23, 60 x 4}: |Q| = 24,
    alpha = 4, dnum = beta = 6, fresh ciphertexts at chain index 1."""
    st = Setup(16, 24, 4, seed=7)
    a, b = st.ct(1), st.ct(1)
    key = st.key()
    out = empty((2, 24, st.N), dev)
    st.ctx.multiply_and_relin(1, to_dev(a, dev), to_dev(b, dev), to_dev(key, dev), out)
    got, want = to_host(out), st.orc.multiply_and_relin(1, a, b, key, threads=8)
    assert np.array_equal(got, want), first_mismatch(got, want)


# (logN, nq, alpha, chain, bits): the fused rescale's last prime in the FP64
# policy (50-bit) and in the integer policy (60-bit), |Ql| = 2 (one limb left)
FUSED_SHAPES = [(logN, nq, alpha, chain, None) for logN, nq, alpha, chain in SHAPES] + [
    (12, 4, 2, 1, [60] * 6),
    (13, 6, 3, 2, [60, 50, 50, 50, 60, 50, 60, 60, 60]),
    (12, 3, 1, 2, None),
]


@pytest.mark.parametrize("logN,nq,alpha,chain,bits", FUSED_SHAPES)
def test_multiply_relin_rescale(dev, logN, nq, alpha, chain, bits):
    """pfa_multiply_relin_rescale equals multiply_and_relin followed by rescale."""
    st = Setup(logN, nq, alpha, seed=11, bits=bits)
    Ql = st.orc.size_Ql(chain)
    a, b = st.ct(chain), st.ct(chain)
    key = st.key()
    out = empty((2, Ql - 1, st.N), dev)
    st.ctx.multiply_relin_rescale(chain, to_dev(a, dev), to_dev(b, dev), to_dev(key, dev), out)
    want = st.orc.rescale(chain, st.orc.multiply_and_relin(chain, a, b, key, threads=8), threads=8)
    got = to_host(out)
    assert np.array_equal(got, want), first_mismatch(got, want)


@pytest.mark.parametrize("logN,nq,alpha,chain,bits", FUSED_SHAPES[:3] + FUSED_SHAPES[-3:])
def test_relinearize_rescale(dev, logN, nq, alpha, chain, bits):
    """pfa_relinearize_rescale equals relinearize followed by rescale."""
    st = Setup(logN, nq, alpha, seed=12, bits=bits)
    Ql = st.orc.size_Ql(chain)
    ct3 = st.ct(chain, 3)
    key = st.key()
    out = empty((2, Ql - 1, st.N), dev)
    st.ctx.relinearize_rescale(chain, to_dev(ct3, dev), to_dev(key, dev), out)
    want = st.orc.rescale(chain, st.orc.keyswitch(chain, ct3[:2], ct3[2], key, threads=8), threads=8)
    got = to_host(out)
    assert np.array_equal(got, want), first_mismatch(got, want)


@pytest.mark.parametrize("logN,nq,alpha,chain", [(12, 20, 1, 1), (12, 18, 1, 2), (13, 34, 2, 1)])
def test_many_digits(dev, logN, nq, alpha, chain):
    """16 or more digits per key switch (long digit loops in the inner
    product): multiply_and_relin and the fused call against the oracle."""
    st = Setup(logN, nq, alpha, seed=14)
    assert st.orc.beta(chain) >= 16
    Ql = st.orc.size_Ql(chain)
    a, b = st.ct(chain), st.ct(chain)
    key = st.key()
    want = st.orc.multiply_and_relin(chain, a, b, key, threads=8)
    out = empty((2, Ql, st.N), dev)
    st.ctx.multiply_and_relin(chain, to_dev(a, dev), to_dev(b, dev), to_dev(key, dev), out)
    got = to_host(out)
    assert np.array_equal(got, want), first_mismatch(got, want)
    fused = empty((2, Ql - 1, st.N), dev)
    st.ctx.multiply_relin_rescale(chain, to_dev(a, dev), to_dev(b, dev), to_dev(key, dev), fused)
    got, want = to_host(fused), st.orc.rescale(chain, want, threads=8)
    assert np.array_equal(got, want), first_mismatch(got, want)


def test_multiply_relin_rescale_config3(dev):
    """The fused path at the benchmark config-3 shape (N = 2^16, |Q| = 24, alpha = 4)."""
    st = Setup(16, 24, 4, seed=13)
    a, b = st.ct(1), st.ct(1)
    key = st.key()
    out = empty((2, 23, st.N), dev)
    st.ctx.multiply_relin_rescale(1, to_dev(a, dev), to_dev(b, dev), to_dev(key, dev), out)
    want = st.orc.rescale(1, st.orc.multiply_and_relin(1, a, b, key, threads=8), threads=8)
    got = to_host(out)
    assert np.array_equal(got, want), first_mismatch(got, want)


@pytest.mark.parametrize("logN", [10, 11, 14, 15, 17])
def test_multiply_tensor_rows_geometries(dev, logN):
    """The HMult's tensor kernel runs the key switch's first INTT pass over d2
    at N <= 2^16 (one kernel per row geometry: 32 rows of 4 threads at N = 2^10,
    2^11, 16 or 8 rows of 16 threads above) and the plain tensor + INTT above:
    multiply_and_relin and multiply_relin_rescale bit-exact against the oracle
    at each, with 60-bit primes (integer policy) in Q."""
    st = Setup(logN, 4, 2, seed=21, bits=[60, 50, 60, 50, 60, 60])
    chain = 1
    a, b, key = st.ct(chain), st.ct(chain), st.key()
    want = st.orc.multiply_and_relin(chain, a, b, key, threads=8)
    out = empty(a.shape, dev)
    st.ctx.multiply_and_relin(chain, to_dev(a, dev), to_dev(b, dev), to_dev(key, dev), out)
    got = to_host(out)
    assert np.array_equal(got, want), first_mismatch(got, want)
    res = empty((2, a.shape[1] - 1, st.N), dev)
    st.ctx.multiply_relin_rescale(chain, to_dev(a, dev), to_dev(b, dev), to_dev(key, dev), res)
    got, want = to_host(res), st.orc.rescale(chain, want, threads=8)
    assert np.array_equal(got, want), first_mismatch(got, want)


def test_multiply_relin_rescale_errors(dev):
    st = Setup(12, 3, 1)
    key = to_dev(st.key(), dev)
    a = to_dev(st.ct(3), dev)
    with pytest.raises(ValueError):  # one limb left: nothing to rescale
        st.ctx.multiply_relin_rescale(3, a, a, key, empty((2, 1, st.N), dev))
    a1 = to_dev(st.ct(1), dev)
    with pytest.raises(ValueError):  # the output may not alias an input
        st.ctx.multiply_relin_rescale(1, a1, a1, key, a1)


@pytest.mark.parametrize("chain,size", [(1, 2), (2, 3), (4, 2)])
def test_rescale(dev, chain, size):
    st = Setup(16, 5, 1, seed=8)
    ct = st.ct(chain, size)
    Ql = st.orc.size_Ql(chain)
    out = empty((size, Ql - 1, st.N), dev)
    st.ctx.rescale(chain, to_dev(ct, dev), out)
    got, want = to_host(out), st.orc.rescale(chain, ct, threads=8)
    assert np.array_equal(got, want), first_mismatch(got, want)


def test_rescale_last_level_rejected(dev):
    st = Setup(12, 3, 1)
    ct = st.ct(3)
    with pytest.raises(ValueError):
        st.ctx.rescale(3, to_dev(ct, dev), empty((2, 1, st.N), dev))


@pytest.mark.parametrize("step", [1, -1, 5, 0, 1000])
def test_galois_ntt(dev, step):
    import pfa_native as P

    st = Setup(16, 4, 1, seed=9)
    elt = P.galois_elt_from_step(step, st.N)
    assert elt == O.elt_from_step(step, st.N)
    x = uniform_limbs(st.rng, (3, st.N), st.mods)
    out = empty((3, st.N), dev)
    st.ctx.apply_galois_ntt(elt, to_dev(x, dev), out, 3)
    assert np.array_equal(to_host(out), st.orc.apply_galois_ntt(x, elt))


@pytest.mark.parametrize("logN,nq,alpha,chain", SHAPES[:4])
def test_apply_galois(dev, logN, nq, alpha, chain):
    import pfa_native as P

    st = Setup(logN, nq, alpha, seed=10)
    ct = st.ct(chain)
    key = st.key()
    elt = P.galois_elt_from_step(3, st.N)
    d = to_dev(ct, dev)
    st.ctx.apply_galois(chain, d, elt, to_dev(key, dev))
    got, want = to_host(d), st.orc.apply_galois(chain, ct, elt, key, threads=8)
    assert np.array_equal(got, want), first_mismatch(got, want)


@pytest.mark.parametrize("logN,nq,alpha,chain", [(12, 6, 2, 1), (12, 5, 1, 2), (16, 6, 3, 1), (17, 3, 1, 1)])
def test_hoist_rotations(dev, logN, nq, alpha, chain):
    import pfa_native as P

    st = Setup(logN, nq, alpha, seed=11)
    ct = st.ct(chain)
    steps = [1, 2, -3, 7]
    elts = [P.galois_elt_from_step(s, st.N) for s in steps]
    keys = [st.key() for _ in steps]
    Ql = st.orc.size_Ql(chain)
    out = empty((len(steps), 2, Ql, st.N), dev)
    st.ctx.hoist_rotations(chain, to_dev(ct, dev), elts, [to_dev(k, dev) for k in keys], out)
    got, want = to_host(out), st.orc.hoist_rotations(chain, ct, elts, keys, threads=8)
    assert np.array_equal(got, want), first_mismatch(got, want)


@pytest.mark.parametrize("logN,nq,alpha", [(12, 6, 2), (12, 5, 1), (13, 8, 4)])
def test_kswitch_key(dev, logN, nq, alpha):
    st = Setup(logN, nq, alpha, seed=12)
    o = st.orc
    new = uniform_limbs(st.rng, (st.QP, st.N), st.mods)
    s = uniform_limbs(st.rng, (st.QP, st.N), st.mods)
    a = uniform_limbs(st.rng, (o.dnum, st.QP, st.N), st.mods)
    e = uniform_limbs(st.rng, (o.dnum, st.QP, st.N), st.mods)
    out = empty((o.dnum, 2, st.QP, st.N), dev)
    st.ctx.kswitch_key(to_dev(new, dev), to_dev(s, dev), to_dev(a, dev), to_dev(e, dev), out)
    assert np.array_equal(to_host(out), o.kswitch_key(new, s, a, e))


def test_poly_elementwise(dev):
    import torch

    st = Setup(12, 4, 2, seed=13)
    L = st.QP
    a = uniform_limbs(st.rng, (L, st.N), st.mods)
    b = uniform_limbs(st.rng, (L, st.N), st.mods)
    da, db, out = to_dev(a, dev), to_dev(b, dev), empty((L, st.N), dev)
    qs = np.array(st.mods, dtype=object)[:, None]
    A, B = a.astype(object), b.astype(object)
    st.ctx.poly_add(da, db, out, L)
    assert np.array_equal(to_host(out).astype(object), (A + B) % qs)
    st.ctx.poly_sub(da, db, out, L)
    assert np.array_equal(to_host(out).astype(object), (A - B) % qs)
    st.ctx.poly_mul(da, db, out, L)
    assert np.array_equal(to_host(out).astype(object), (A * B) % qs)
    st.ctx.poly_negate(da, out, L)
    assert np.array_equal(to_host(out).astype(object), (-A) % qs)
    v = st.rng.integers(-(2 ** 62), 2 ** 62, size=st.N, dtype=np.int64)
    v[:4] = [0, -1, np.iinfo(np.int64).min, np.iinfo(np.int64).max]
    st.ctx.poly_from_signed(torch.from_numpy(v).to(dev), out, L)
    want = np.array([[int(x) % q for x in v] for q in st.mods], dtype=object)
    assert np.array_equal(to_host(out).astype(object), want)


def test_key_too_short_rejected(dev):
    st = Setup(12, 6, 2)
    ct = st.ct(1)
    key = uniform_limbs(st.rng, (2, 2, st.QP, st.N), st.mods)  # dnum 2 < beta 3
    with pytest.raises(ValueError):
        st.ctx.keyswitch(1, to_dev(ct, dev), to_dev(ct[1], dev), to_dev(key, dev))


def test_top_level_of_uneven_chain_rejected(dev):
    """|Q| = 7, alpha = 2: keys have dnum = 3 digits (src/secretkey.cu:366) but the top
    level needs beta = 4; the reference would read past its key array, here it is an error
    (and the oracle refuses it too)."""
    st = Setup(12, 7, 2)
    ct = st.ct(1)
    key = st.key()
    with pytest.raises(ValueError):
        st.ctx.keyswitch(1, to_dev(ct, dev), to_dev(ct[1], dev), to_dev(key, dev))
    with pytest.raises(ValueError):
        st.orc.keyswitch(1, ct, ct[1], key)


@pytest.mark.parametrize("slots", [64, 48, 40, 16])
@pytest.mark.parametrize("logN,nq,alpha,chain", [(12, 9, 3, 1), (12, 20, 1, 1), (13, 12, 4, 1)])
def test_inner_product_split_items(dev, monkeypatch, slots, logN, nq, alpha, chain):
    """The inner product splits the items left over after whole rounds of its
    resident workgroups into digit chunks whose partial sums the last chunk
    adds (k_inner_ws).  PFA_WS_SLOTS shrinks the assumed resident count so small
    shapes split with several chunk counts; the fused and two-call HMult and the
    key switch stay bit-exact against the oracle, and no placement error is
    recorded."""
    monkeypatch.setenv("PFA_WS_SLOTS", str(slots))
    st = Setup(logN, nq, alpha, seed=slots + logN)
    Ql = st.orc.size_Ql(chain)
    a, b = st.ct(chain), st.ct(chain)
    key = st.key()
    want = st.orc.multiply_and_relin(chain, a, b, key, threads=8)
    out = empty((2, Ql, st.N), dev)
    st.ctx.multiply_and_relin(chain, to_dev(a, dev), to_dev(b, dev), to_dev(key, dev), out)
    got = to_host(out)
    assert np.array_equal(got, want), first_mismatch(got, want)
    fused = empty((2, Ql - 1, st.N), dev)
    st.ctx.multiply_relin_rescale(chain, to_dev(a, dev), to_dev(b, dev), to_dev(key, dev), fused)
    got, want_r = to_host(fused), st.orc.rescale(chain, want, threads=8)
    assert np.array_equal(got, want_r), first_mismatch(got, want_r)
    st.ctx.synchronize()


@pytest.mark.parametrize("slots", [0, 40])
@pytest.mark.parametrize("logN,nq,alpha,chain,bits", [(12, 9, 3, 1, None), (12, 4, 2, 1, [60] * 6),
                                                      (13, 6, 3, 2, [60, 50, 50, 50, 60, 50, 60, 60, 60])])
def test_multiply_batches(dev, monkeypatch, slots, logN, nq, alpha, chain, bits):
    """pfa_multiply_and_relin_batch and pfa_multiply_relin_rescale_batch over 3
    pairs: every member bit-exact against the oracle's multiply_and_relin (and
    rescale) of its pair, with whole and (PFA_WS_SLOTS = 40) split inner-product
    items, whose split chunks then carry the fold of other members."""
    if slots:
        monkeypatch.setenv("PFA_WS_SLOTS", str(slots))
    st = Setup(logN, nq, alpha, seed=21 + slots, bits=bits)
    Ql = st.orc.size_Ql(chain)
    K = 3
    a = np.stack([st.ct(chain) for _ in range(K)])
    b = np.stack([st.ct(chain) for _ in range(K)])
    key = st.key()
    da, db, dk = to_dev(a, dev), to_dev(b, dev), to_dev(key, dev)
    want = [st.orc.multiply_and_relin(chain, a[i], b[i], key, threads=8) for i in range(K)]
    out = empty((K, 2, Ql, st.N), dev)
    st.ctx.multiply_and_relin_batch(chain, K, da, db, dk, out)
    got = to_host(out)
    for i in range(K):
        assert np.array_equal(got[i], want[i]), (i, first_mismatch(got[i], want[i]))
    res = empty((K, 2, Ql - 1, st.N), dev)
    st.ctx.multiply_relin_rescale_batch(chain, K, da, db, dk, res)
    got = to_host(res)
    for i in range(K):
        w = st.orc.rescale(chain, want[i], threads=8)
        assert np.array_equal(got[i], w), (i, first_mismatch(got[i], w))
    # in place: out = a
    st.ctx.multiply_and_relin_batch(chain, K, da, db, dk, da)
    got = to_host(da)
    for i in range(K):
        assert np.array_equal(got[i], want[i]), (i, first_mismatch(got[i], want[i]))
    st.ctx.synchronize()


def test_multiply_batch_errors(dev):
    st = Setup(12, 4, 2)
    a = to_dev(np.stack([st.ct(1), st.ct(1)]), dev)
    key = to_dev(st.key(), dev)
    with pytest.raises(ValueError):
        st.ctx.multiply_relin_rescale_batch(1, 2, a, a, key, a)  # output overlaps an input
    with pytest.raises(ValueError):
        st.ctx.multiply_and_relin_batch(1, 0, a, a, key, a)  # empty batch


@pytest.mark.parametrize("slots", [0, 40])
@pytest.mark.parametrize("logN,nq,alpha,chain", [(12, 6, 2, 1), (12, 5, 1, 2), (13, 6, 3, 1)])
def test_rotate_batch(dev, monkeypatch, slots, logN, nq, alpha, chain):
    """pfa_rotate_batch: 3 ciphertexts, each with its own Galois element and
    key, every member bit-exact against the oracle's apply_galois (whole and
    split inner-product items)."""
    import pfa_native as P

    if slots:
        monkeypatch.setenv("PFA_WS_SLOTS", str(slots))
    st = Setup(logN, nq, alpha, seed=30 + slots)
    cts = np.stack([st.ct(chain) for _ in range(3)])
    keys = [st.key() for _ in range(3)]
    elts = [P.galois_elt_from_step(s, st.N) for s in (1, -5, 7)]
    out = empty(cts.shape, dev)
    st.ctx.rotate_batch(chain, to_dev(cts, dev), elts, [to_dev(k, dev) for k in keys], out)
    got = to_host(out)
    for i in range(3):
        want = st.orc.apply_galois(chain, cts[i], elts[i], keys[i], threads=8)
        assert np.array_equal(got[i], want), (i, first_mismatch(got[i], want))
