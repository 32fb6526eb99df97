"""CPU checks of the bootstrapping plan (no GPU): the host-side pieces that the
GPU pipeline is built from, each pinned by mathematics rather than by
restating the formula.

* CoeffToSlot / SlotToCoeff layers (src/bootstrap.cu:256-437): the product of
  the layers' diagonal matrices is compared with the canonical embedding
  E[j][k] = zeta^(5^j k), built directly from its definition: C2S E must be the
  bit-reversal permutation and S2C the inverse of C2S.
* EvalMod polynomial (the role of src/evalmod.cu): the Chebyshev fit plus r
  double angles must equal sin(2 pi x) / (2 pi) ~ x - round(x) on the domain
  |x| < K, within the error budget the 1e-3 post-bootstrap tolerance
  (test/ckks_engine_test.cu:182) leaves.
* The Paterson-Stockmeyer split T_m hi + lo equals the polynomial it splits.
* The oracle's ModRaise (src/bootstrap.cu:37-75) against Python integers,
  including the boundary residue floor(q0 / 2), which the reference reads as
  negative.
"""
import numpy as np
import pytest
from numpy.polynomial import chebyshev as C

import py_oracle as O
import pyPhantom as ph


def dense(diags, n):
    A = np.zeros((n, n), complex)
    r = np.arange(n)
    for d, v in diags.items():
        A[r, (r + d) % n] += v
    return A


def embedding(N):
    n, M = N // 2, 2 * N
    rot = np.array([pow(5, j, M) for j in range(n)])
    k = np.arange(n)
    return np.exp(1j * np.pi * ((rot[:, None] * k[None, :]) % M) / N)


def brv_perm(n):
    bits = n.bit_length() - 1
    P = np.zeros((n, n))
    for j in range(n):
        P[j, ph._brv_index(j, bits)] = 1
    return P


@pytest.mark.parametrize("logN,stages", [(6, [2, 2, 1]), (7, [2, 2, 2]), (8, [3, 3, 1])])
def test_c2s_layers_invert_the_embedding(logN, stages):
    N = 1 << logN
    n = N // 2
    c2s = ph.build_c2s_diagonals(logN, stages)
    s2c = ph.build_s2c_diagonals(logN, stages)
    A = np.eye(n)
    for L in c2s.layers:
        A = dense(L, n) @ A
    B = np.eye(n)
    for L in s2c.layers:
        B = dense(L, n) @ B
    E, P = embedding(N), brv_perm(n)
    assert np.max(np.abs(A @ E - P)) < 1e-12
    assert np.max(np.abs(B @ P - E)) < 1e-12
    assert np.max(np.abs(B @ A - np.eye(n))) < 1e-12


@pytest.mark.parametrize("logN,stages", [(8, [3, 3, 1]), (12, [4, 4, 3])])
def test_layer_diagonals_and_rotations(logN, stages):
    N = 1 << logN
    lt = ph.build_c2s_diagonals(logN, stages)
    elts = set(ph.bootstrap_required_galois_elts(logN, stages))
    assert 2 * N - 1 in elts
    for i, g in enumerate(stages):
        assert len(lt.layers[i]) <= 2 ** (g + 1) - 1
        assert all(d % lt.units[i] == 0 for d in lt.layers[i])
        n1, groups, _ = lt.baby_giant(i)
        for G, terms in groups.items():
            for b, d in terms:
                assert (G * n1 + b) * lt.units[i] == d
                if b:
                    assert ph.get_elt_from_step(b * lt.units[i], N) in elts
            if G:
                assert ph.get_elt_from_step(ph._signed_step(G * n1 * lt.units[i], N // 2), N) in elts


def test_evalmod_polynomial_is_the_modular_sine():
    K, r, deg = ph.BOOT_K, ph.BOOT_R, ph.BOOT_DEG
    c = ph.evalmod_chebyshev(K, r, deg)
    rng = np.random.default_rng(5)
    I = rng.integers(-K + 1, K, 100000)
    dq = 2.0 ** -20                       # user scale / q0 of the bootstrap chain
    m = rng.uniform(-3, 3, I.size)
    x = I + dq * m
    y = C.chebval(x / K, c)
    for _ in range(r):
        y = 2 * y * y - 1
    y /= 2 * np.pi
    assert np.max(np.abs(y - np.sin(2 * np.pi * x) / (2 * np.pi))) < 1e-13
    assert np.max(np.abs(y / dq - m)) < 2e-7   # message units


def test_chebyshev_split_reassembles():
    rng = np.random.default_rng(9)
    t = np.linspace(-1, 1, 257)
    for deg in (8, 15, 40, 63):
        c = list(rng.standard_normal(deg + 1))
        m, hi, lo = ph._cheb_split(c)
        Tm = C.chebval(t, [0] * m + [1])
        assert np.allclose(C.chebval(t, c), Tm * C.chebval(t, hi) + C.chebval(t, lo), atol=1e-10)
        assert len(hi) - 1 == deg - m and len(lo) == m


def test_cheb_depth():
    assert [ph._cheb_depth(d) for d in (1, 2, 3, 7, 8, 15, 31, 63)] == [1, 2, 3, 4, 4, 5, 6, 7]
    assert ph._cheb_depth(ph.BOOT_DEG) + ph.BOOT_R == ph.BOOT_EVALMOD_LEVELS


def test_oracle_mod_raise_centres():
    N = 64
    mods = O.create_coeff_modulus(N, [60, 50, 40, 60])
    orc = O.Oracle(N, mods, 1)
    q0 = mods[0]
    rng = np.random.default_rng(3)
    coef = [int(v) for v in rng.integers(0, q0, N, dtype=np.uint64)]
    coef[:4] = [0, q0 >> 1, (q0 >> 1) - 1, q0 - 1]
    ct = orc.ntt_fwd(np.array(coef, dtype=np.uint64).reshape(1, 1, N))
    got = orc.ntt_inv(orc.mod_raise(ct, 3))
    for l in range(3):
        q = mods[l]
        want = [(v - q0 if v >= q0 >> 1 else v) % q for v in coef]
        assert [int(v) for v in got[0, l]] == want


@pytest.mark.parametrize("variant,bound", [("k7_r3", 1e-5), ("k16_r3", 2e-9), ("k28_r3", 1e-9)])
def test_reference_evalmod_polynomials(variant, bound):
    """The reference's EvalMod polynomials (src/evalmod.cu tables, PS
    factorings and double angles), evaluated in float64 by the same operation
    sequence pyPhantom runs on ciphertexts, approximate sin(2 pi K x) / (2 pi)
    on [-1, 1] to the precision the reference states for them (K = 7 ~17 bits
    observed 6e-6, K = 16 and K = 28 30+ bits; test/evalmod_test.cu:209-216).
    A wrong table entry, basis recurrence or factoring step breaks this by
    orders of magnitude."""
    K = ph.EVALMOD_K[variant]
    x = np.linspace(-1.0, 1.0, 200001)
    err = np.abs(ph.evalmod_model(x, variant) - np.sin(2 * np.pi * K * x) / (2 * np.pi))
    assert err.max() < bound, err.max()


def test_reference_evalmod_k28_r4_is_not_the_sine():
    """evalmod_k28_r4 runs the K = 28 polynomial tuned for three double angles
    through four; the reference documents the result as off by ~0.1 and keeps
    the variant out of its test (test/evalmod_test.cu:236-243).  The model
    shows the same."""
    x = np.linspace(-1.0, 1.0, 20001)
    err = np.abs(ph.evalmod_model(x, "k28_r4") - np.sin(2 * np.pi * 28 * x) / (2 * np.pi))
    assert err.max() > 0.1


def test_evalmod_levels_match_the_reference():
    """Levels consumed (include/evalmod.h): K = 7 eight, K = 16 and K = 28 nine,
    K = 28 R = 4 ten -- the depth of the evaluation graph, counted here by
    running the model on integers that count rescales."""
    class Depth:
        def __init__(self, d):
            self.d = d

        def __mul__(self, o):
            return Depth(max(self.d, o.d) + 1) if isinstance(o, Depth) else self

        __rmul__ = __mul__

        def __add__(self, o):
            return Depth(max(self.d, o.d)) if isinstance(o, Depth) else self

        __radd__ = __add__

        def __sub__(self, o):
            return self + o

        def __neg__(self):
            return self

    class Ops(ph._EvalModOps):
        def weighted_sum(self, basis, coeffs):
            return Depth(max(b.d for b in basis) + 1)

    for v, levels in ph.EVALMOD_LEVELS.items():
        ops = Ops(None, 1.0)
        out = ph._double_angle(ops, ph._sine(ops, Depth(0), v), ph.EVALMOD_R[v])
        assert out.d == levels, (v, out.d)
