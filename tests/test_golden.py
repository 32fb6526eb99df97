"""The CPU oracle and the library's host-side prime search reproduce the
committed golden vectors (tests/golden/make_golden.py computes them in plain
Python integers from the reference's definitions, sharing no code with either)."""
import numpy as np
import pytest

import py_oracle as O
from golden_data import N, golden, ints

PRIME_SETS = {
    "c1_n8192": (8192, [50, 50, 55, 60]),
    "c2_n65536": (65536, [50] * 35 + [60]),
    "c3_n65536": (65536, [60] + [50] * 23 + [60] * 4),
    "c4_n65536": (65536, [60] + [40] * 19 + [60] * 4),
}


@pytest.mark.parametrize("name", sorted(PRIME_SETS))
def test_primes_oracle_and_library(name):
    import pfa_native as P

    n, bits = PRIME_SETS[name]
    want = ints(golden()[f"primes_{name}"])
    assert O.create_coeff_modulus(n, bits) == want
    assert P.create_coeff_modulus(n, bits) == want


def test_config1_roots():
    g = golden()
    mods = ints(g["primes_c1_n8192"])
    orc = O.Oracle(8192, mods, 1)
    assert [orc.root(i) for i in range(len(mods))] == ints(g["roots_c1_n8192"])


def test_ntt_vectors():
    g = golden()
    mods = ints(g["ntt_moduli"])
    orc = O.Oracle(N, mods, 1)
    assert [orc.root(i) for i in range(4)] == ints(g["ntt_roots"])
    assert np.array_equal(orc.ntt_fwd(g["ntt_in"]), g["ntt_out"])
    assert np.array_equal(orc.ntt_inv(g["ntt_out"]), g["ntt_in"])


def test_galois_vectors():
    g = golden()
    for step, elt, perm in zip(g["galois_steps"], g["galois_elts"], g["galois_perms"]):
        assert O.elt_from_step(int(step), N) == int(elt)
        assert np.array_equal(O.galois_perm(N, int(elt)), perm)


def _ks_oracle():
    g = golden()
    return g, O.Oracle(N, ints(g["ks_moduli"]), int(g["ks_alpha"]))


def test_keyswitch_chain_vectors():
    g, orc = _ks_oracle()
    assert [orc.root(i) for i in range(6)] == ints(g["ks_roots"])
    assert np.array_equal(orc.tensor(g["ks_a"], g["ks_b"]), g["ks_tensor"])
    assert np.array_equal(orc.modup(1, g["ks_tensor"][2]), g["ks_modup"])
    assert np.array_equal(orc.modup(2, g["ks_c2_low"]), g["ks_modup_low"])
    assert np.array_equal(orc.ks_inner_prod(1, g["ks_modup"], g["ks_key"]), g["ks_cx"])
    for k in range(2):
        assert np.array_equal(orc.moddown(1, g["ks_cx"][k]), g["ks_moddown"][k])
    assert np.array_equal(orc.multiply_and_relin(1, g["ks_a"], g["ks_b"], g["ks_key"]), g["ks_mul_relin"])
    assert np.array_equal(orc.rescale(1, g["ks_mul_relin"]), g["ks_rescale"])


def test_golden_catches_a_planted_mistake():
    """A one-residue change in an oracle output is seen by the vector comparison."""
    g, orc = _ks_oracle()
    got = orc.rescale(1, g["ks_mul_relin"])
    q = int(g["ks_moduli"][1])
    got[1, 1, 7] = (int(got[1, 1, 7]) + 1) % q
    assert not np.array_equal(got, g["ks_rescale"])


def test_rotation_vectors():
    """apply_galois permutes c1 before the key switch (src/evaluate.cu:1607-1656);
    hoist_rotations permutes the ModUp slabs (:2036-2045); hoisting sums the
    rotations' inner products before one ModDown (:1732-1925).  The oracle
    reproduces each order's vectors, and the two orders' residues differ."""
    g, orc = _ks_oracle()
    elts = ints(g["rot_elts"])
    keys = list(g["rot_keys"])
    ag = orc.apply_galois(1, g["rot_ct"], elts[0], keys[0])
    assert np.array_equal(ag, g["rot_apply_galois"])
    hr = orc.hoist_rotations(1, g["rot_ct"], elts, keys)
    assert np.array_equal(np.stack(hr), g["rot_hoist_rotations"])
    assert not np.array_equal(hr[0], ag)
    hs = orc.hoisting(2, g["hoisting_ct"], ints(g["hoisting_elts"]), list(g["hoisting_keys"]))
    assert np.array_equal(hs, g["hoisting_out"])
