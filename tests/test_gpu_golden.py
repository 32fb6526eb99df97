"""The HIP path reproduces the committed golden vectors (tests/golden/), bit for bit."""
import numpy as np
import pytest

import pfa_native as P
from golden_data import N, golden, ints
from gpu_util import empty, first_mismatch, to_dev, to_host

pytestmark = pytest.mark.gpu


def _eq(got, want, what):
    assert np.array_equal(got, want), f"{what}: {first_mismatch(got, want)}"


def test_ntt_vectors(dev):
    g = golden()
    ctx = P.NativeContext(N, ints(g["ntt_moduli"]), 1)
    try:
        assert ctx.roots() == ints(g["ntt_roots"])
        d = to_dev(g["ntt_in"], dev)
        ctx.ntt_forward(d, 1, 4, 0)
        _eq(to_host(d), g["ntt_out"], "forward NTT")
        ctx.ntt_inverse(d, 1, 4, 0)
        _eq(to_host(d), g["ntt_in"], "inverse NTT")
    finally:
        ctx.close()


def test_galois_vectors(dev):
    g = golden()
    ctx = P.NativeContext(N, ints(g["ntt_moduli"]), 1)
    try:
        src = g["ntt_out"]
        for elt, perm in zip(g["galois_elts"], g["galois_perms"]):
            out = empty(src.shape, dev)
            ctx.apply_galois_ntt(int(elt), to_dev(src, dev), out, 4)
            _eq(to_host(out), src[:, perm.astype(np.int64)], f"Galois elt {int(elt)}")
    finally:
        ctx.close()


def test_keyswitch_chain_vectors(dev):
    g = golden()
    ctx = P.NativeContext(N, ints(g["ks_moduli"]), int(g["ks_alpha"]))
    try:
        assert ctx.roots() == ints(g["ks_roots"])
        a, b, key = (to_dev(g[k], dev) for k in ("ks_a", "ks_b", "ks_key"))
        t = empty((3, 4, N), dev)
        ctx.tensor(1, a, b, t)
        _eq(to_host(t), g["ks_tensor"], "tensor")
        up = empty((2, 6, N), dev)
        ctx.modup(1, to_dev(g["ks_tensor"][2], dev), up)
        _eq(to_host(up), g["ks_modup"], "ModUp")
        up_low = empty((2, 5, N), dev)
        ctx.modup(2, to_dev(g["ks_c2_low"], dev), up_low)
        _eq(to_host(up_low), g["ks_modup_low"], "ModUp at chain index 2")
        cx = empty((2, 6, N), dev)
        ctx.ks_inner_prod(1, to_dev(g["ks_modup"], dev), key, cx)
        _eq(to_host(cx), g["ks_cx"], "inner product")
        for k in range(2):
            md = empty((4, N), dev)
            ctx.moddown(1, to_dev(g["ks_cx"][k], dev), md)
            _eq(to_host(md), g["ks_moddown"][k], f"ModDown poly {k}")
        out = empty((2, 4, N), dev)
        ctx.multiply_and_relin(1, a, b, key, out)
        _eq(to_host(out), g["ks_mul_relin"], "multiply_and_relin")
        res = empty((2, 3, N), dev)
        ctx.rescale(1, out, res)
        _eq(to_host(res), g["ks_rescale"], "rescale")
    finally:
        ctx.close()


def test_rotation_vectors(dev):
    """The rotation orders of the reference: apply_galois (permute c1, then
    key-switch), hoist_rotations (ModUp once, permute the slabs) and hoisting
    (summed inner products, one ModDown), bit for bit."""
    g = golden()
    ctx = P.NativeContext(N, ints(g["ks_moduli"]), int(g["ks_alpha"]))
    try:
        elts = ints(g["rot_elts"])
        keys = [to_dev(k, dev) for k in g["rot_keys"]]
        d = to_dev(g["rot_ct"], dev)
        ctx.apply_galois(1, d, elts[0], keys[0])
        _eq(to_host(d), g["rot_apply_galois"], "apply_galois")
        out = empty((len(elts), 2, 4, N), dev)
        ctx.hoist_rotations(1, to_dev(g["rot_ct"], dev), elts, keys, out)
        _eq(to_host(out), g["rot_hoist_rotations"], "hoist_rotations")
        hs = empty((2, 3, N), dev)
        ctx.hoisting(2, to_dev(g["hoisting_ct"], dev), ints(g["hoisting_elts"]),
                     [to_dev(k, dev) for k in g["hoisting_keys"]], hs)
        _eq(to_host(hs), g["hoisting_out"], "hoisting")
    finally:
        ctx.close()
