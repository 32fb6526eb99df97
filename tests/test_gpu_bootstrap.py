"""GPU tests of CKKS bootstrapping (src/bootstrap.cu:1703-1951).

* pfa_mod_raise is bit-exact against the oracle's restatement of
  mod_raise_signed_tile_kernel (src/bootstrap.cu:37-75), itself pinned against
  Python integers in tests/test_bootstrap_math.py.
* pfa_ct_lincomb (the integer-weighted sums of EvalMod) is bit-exact against
  Python integers.
* Every CoeffToSlot / SlotToCoeff layer is bit-exact against the oracle
  running the same rotations, diagonal products, sums and rescale.
* End to end, the reference's acceptance test is the bar: decoded slots after
  bootstrap within 1e-3 of the input (test/ckks_engine_test.cu:182-188); the
  refreshed ciphertext must also take a further multiplication.
"""
import numpy as np
import pytest

import py_oracle as O
from gpu_util import empty, to_dev, to_host

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("logN,bits,special", [(12, [60, 40, 40, 50, 60, 60], 2), (16, None, 6)])
def test_mod_raise_matches_oracle(dev, logN, bits, special):
    """At N = 2^12 and on config 5's chain at N = 2^16 (30 primes + 6 special)."""
    import pfa_native as P
    import pyPhantom as ph

    N = 1 << logN
    mods = O.create_coeff_modulus(N, bits or ph.bootstrap_coeff_bits())
    ctx = P.NativeContext(N, mods, special)
    orc = O.Oracle(N, mods, special)
    q0 = mods[0]
    rng = np.random.default_rng(21)
    coef = rng.integers(0, q0, (2, 1, N), dtype=np.uint64)
    coef[0, 0, :4] = [0, q0 >> 1, (q0 >> 1) - 1, q0 - 1]
    ct = orc.ntt_fwd(coef)
    Q = len(mods) - special
    out = empty((2, Q, N), dev)
    ctx.mod_raise(to_dev(ct, dev), out)
    got, want = to_host(out), orc.mod_raise(ct, Q)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("bias", [None, 0, (1 << 119) + 12345, -(1 << 126) + 7])
def test_ct_lincomb_matches_integers(dev, bias):
    """pfa_ct_lincomb against Python integers: inputs at several limb counts,
    signed constants up to the int64 ends, signed 128-bit biases."""
    import pfa_native as P

    N = 1 << 12
    mods = O.create_coeff_modulus(N, [60, 40, 50, 60, 60, 60])
    ctx = P.NativeContext(N, mods, 1)
    rng = np.random.default_rng(31)
    L = 3
    limbs = [3, 5, 4, 3]
    ins = [np.stack([np.stack([rng.integers(0, q, N, dtype=np.uint64) for q in mods[:Lt]]) for _ in range(2)])
           for Lt in limbs]
    consts = [2, -(1 << 63), (1 << 63) - 1, -987654321987]
    out = empty((2, L, N), dev)
    ctx.ct_lincomb(L, [to_dev(x, dev) for x in ins], consts, out, bias)
    got = to_host(out)
    for k in range(2):
        for l in range(L):
            q = mods[l]
            acc = [0] * N
            for x, c in zip(ins, consts):
                row = x[k, l].tolist()
                acc = [(a + c * v) for a, v in zip(acc, row)]
            if k == 0 and bias is not None:
                acc = [a + bias for a in acc]
            assert got[k, l].tolist() == [a % q for a in acc], (k, l)


def test_ct_lincomb_bias_per_ciphertext(dev):
    """With ct_size = 2 over 4 polys (a bundle of two ciphertexts) the bias
    goes to polys 0 and 2 only."""
    import pfa_native as P

    N = 1 << 12
    mods = O.create_coeff_modulus(N, [60, 40, 60])
    ctx = P.NativeContext(N, mods, 1)
    rng = np.random.default_rng(6)
    x = np.stack([np.stack([rng.integers(0, q, N, dtype=np.uint64) for q in mods[:2]]) for _ in range(4)])
    out = empty((4, 2, N), dev)
    bias = -(1 << 100) + 3
    ctx.ct_lincomb(2, [to_dev(x, dev)], [7], out, bias, ct_size=2)
    got = to_host(out)
    for k in range(4):
        for l in range(2):
            q = mods[l]
            want = [(7 * v + (bias if k % 2 == 0 else 0)) % q for v in x[k, l].tolist()]
            assert got[k, l].tolist() == want, (k, l)


def test_ct_lincomb_in_place(dev):
    import pfa_native as P

    N = 1 << 12
    mods = O.create_coeff_modulus(N, [60, 40, 60])
    ctx = P.NativeContext(N, mods, 1)
    rng = np.random.default_rng(5)
    x = np.stack([np.stack([rng.integers(0, q, N, dtype=np.uint64) for q in mods[:2]]) for _ in range(2)])
    t = to_dev(x, dev)
    ctx.ct_lincomb(2, [t], [-3], t, -5)
    got = to_host(t)
    for k in range(2):
        for l in range(2):
            q = mods[l]
            assert got[k, l].tolist() == [(-3 * v - (5 if k == 0 else 0)) % q for v in x[k, l].tolist()]


def boot_setup(logN, user_levels, special, seed=4):
    import pyPhantom as ph

    N = 1 << logN
    stages = ph._default_stages(logN)
    p = ph.params(ph.scheme_type.ckks)
    p.set_poly_modulus_degree(N)
    p.set_coeff_modulus(ph.create_coeff_modulus(N, ph.bootstrap_coeff_bits(user_levels, special=special)))
    p.set_special_modulus_size(special)
    p.set_galois_elts(ph.bootstrap_required_galois_elts(logN, stages))
    ctx = ph.context(p)
    sk = ph.secret_key(ctx, seed=seed)
    enc = ph.ckks_encoder(ctx)
    bk = ph.create_bootstrap_key(ctx, enc, sk, sparse_hamming_weight=192, seed=seed + 1, evalmod="cheb63")
    return ph, ctx, sk, enc, bk


@pytest.fixture(scope="module")
def boot12(dev):
    return boot_setup(12, 3, 4)


@pytest.mark.parametrize("kind", ["real", "complex"])
def test_bootstrap_refreshes(boot12, kind):
    ph, ctx, sk, enc, bk = boot12
    n = enc.slot_count()
    rng = np.random.default_rng(7)
    z = rng.uniform(-1, 1, n)
    if kind == "complex":
        z = z + 1j * rng.uniform(-1, 1, n)
    scale = 2.0 ** 40
    bottom = ctx.size_Q
    ct = sk.encrypt_symmetric(ctx, enc.encode_complex_vector(ctx, z, scale, bottom), seed=8)
    out = ph.bootstrap(ctx, enc, ct, bk, scale)
    assert out.chain_index() == 1 + 2 * 3 + ph.BOOT_EVALMOD_LEVELS
    got = np.array(enc.decode_complex_vector(ctx, sk.decrypt(ctx, out)))
    err = np.max(np.abs(got - z))
    print(f"bootstrap N=2^12 {kind}: max |err| {err:.3e} ({-np.log2(err):.1f} bits)")
    assert err < 1e-3
    # the refreshed ciphertext takes a further multiplication
    sq = ph.rescale_to_next(ctx, ph.multiply_and_relin(ctx, out, out, bk.rlk))
    got2 = np.array(enc.decode_complex_vector(ctx, sk.decrypt(ctx, sq)))
    assert np.max(np.abs(got2 - z * z)) < 4e-3


def test_mod_raise_api_keeps_message(boot12):
    """mod_raise_inplace through the encapsulation keys: the raised ciphertext
    decrypts to m + q0 I with I small and integral."""
    ph, ctx, sk, enc, bk = boot12
    z = np.random.default_rng(2).uniform(-1, 1, enc.slot_count())
    ct = sk.encrypt_symmetric(ctx, enc.encode_double_vector(ctx, z, 2.0 ** 40, ctx.size_Q), seed=3)
    raised = ph.mod_raise_inplace(ctx, ct, bk.small)
    assert raised.chain_index() == 1
    # reading the raised plaintext at scale 2^40 after dropping all primes but
    # q0 gives the message back
    low = ph.mod_switch_to(ctx, raised, ctx.size_Q)
    got = np.array(enc.decode_double_vector(ctx, sk.decrypt(ctx, low)))
    assert np.max(np.abs(got - z)) < 1e-6


def test_bootstrap_cheb63_options(boot12):
    """This build's EvalMod pipeline takes its own level count and returns the
    message at the input scale: the reference's layout options are refused
    for it, not ignored (python/src/binding.cu:320-336)."""
    ph, ctx, sk, enc, bk = boot12
    with pytest.raises(ValueError):
        ph.create_bootstrap_key(ctx, enc, sk, sparse_hamming_weight=192, eval_mod_levels=9, evalmod="cheb63")
    with pytest.raises(ValueError):
        ph.create_bootstrap_key(ctx, enc, sk, sparse_hamming_weight=192, user_scale=2.0 ** 40, evalmod="cheb63")
    with pytest.raises(ValueError):
        ph.create_bootstrap_key(ctx, enc, sk, sparse_hamming_weight=192, split_scale_down=True, evalmod="cheb63")
    z = np.zeros(enc.slot_count())
    ct = sk.encrypt_symmetric(ctx, enc.encode_double_vector(ctx, z, 2.0 ** 40, ctx.size_Q), seed=1)
    with pytest.raises(ValueError):
        ph.bootstrap(ctx, enc, ct, bk, 2.0 ** 40, split_scale_down=True)


def test_cheb63_evalmod_bundle_matches_tracks(boot12):
    """This build's EvalMod on a bundle of two ciphertexts (bootstrap's real and
    imaginary tracks) is bit-identical to EvalMod of each alone."""
    ph, ctx, sk, enc, bk = boot12
    rng = np.random.default_rng(9)
    chain = 5  # past ModRaise, CoeffToSlot's layers and the conjugate split
    q0 = float(ctx.moduli[0])  # EvalMod's input scale in bootstrap
    cts = [sk.encrypt_symmetric(ctx, enc.encode_double_vector(ctx, rng.uniform(-1, 1, enc.slot_count()) / 8,
                                                              q0, chain), seed=10 + i) for i in range(2)]
    alone = [ph._eval_mod(ctx, c, bk) for c in cts]
    both = ph._unbundle(ph._eval_mod(ctx, ph._bundle(ctx, cts), bk))
    for a, b in zip(alone, both):
        assert a.chain_index() == b.chain_index() and a.scale() == b.scale()
        assert bool((a.data == b.data).all())


def _oracle_layer(orc, ph, N, chain, ct, lt, plan, i, keys):
    """One transform layer (hoisted baby rotations, the diagonal products, the
    giant rotations, their sum, the rescale) run operation by operation on the
    oracle: rotations by apply_galois / hoist_rotations (src/evaluate.cu:1607-1656,
    :2041-2045), products by mul_poly, sums mod q."""
    n1, _, _ = lt.baby_giant(i)
    unit = lt.units[i]
    qs = orc.moduli[:orc.size_Ql(chain)]
    rot = {0: ct}
    moved = [b for b in plan.babies if b]
    if moved:
        elts = [ph.get_elt_from_step(b * unit, N) for b in moved]
        for b, r in zip(moved, orc.hoist_rotations(chain, ct, elts, [keys[e] for e in elts], threads=8)):
            rot[b] = r
    M = len(plan.babies)
    acc = np.zeros_like(ct)
    for g, step in enumerate(plan.giants):
        part = np.zeros_like(ct)
        for bi, b in enumerate(plan.babies):
            pt = to_host(plan.grid[g * M + bi])
            for k in range(2):
                part[k] = _add_mod(part[k], orc.mul_poly(pt, rot[b][k]), qs)
        if step:
            e = ph.get_elt_from_step(ph._signed_step(step * n1 * unit, lt.n), N)
            part = orc.apply_galois(chain, part, e, keys[e], threads=8)
        acc = _add_mod(acc, part, qs)
    return orc.rescale(chain, acc, threads=8)


def _add_mod(a, b, qs):
    out = a + b  # residues below 2^61: no uint64 overflow
    for l, q in enumerate(qs):
        out[..., l, :] %= np.uint64(q)
    return out


def test_transform_layers_match_oracle(boot12):
    """Every layer of CoeffToSlot and SlotToCoeff, as bootstrap runs them
    (_apply_layer: one hoisted ModUp for the babies, pfa_bsgs_mac for the
    diagonal products, the giants as one batched rotation, one weighted sum,
    the rescale), has the residues of the oracle running the same operations
    one by one on the same diagonals.  The inputs are fresh encryptions at the
    layers' levels (the residue algebra does not depend on the message)."""
    ph, ctx, sk, enc, bk = boot12
    orc = O.Oracle(ctx.N, ctx.moduli, ctx.size_P)
    keys = {e: to_host(k) for e, k in bk.glk.keys.items()}
    rng = np.random.default_rng(21)
    cases = [(bk.c2s, bk.c2s_pts, i, 1 + i) for i in range(len(bk.c2s_pts))]
    cases += [(bk.s2c, bk.s2c_pts, i, bk.s2c_start + i) for i in range(len(bk.s2c_pts))]
    rotations = 0
    for n, (lt, pts, i, chain) in enumerate(cases):
        plan = pts[i]
        rotations += sum(1 for b in plan.babies if b) + sum(1 for g in plan.giants if g)
        z = rng.uniform(-1, 1, enc.slot_count()) + 1j * rng.uniform(-1, 1, enc.slot_count())
        ct = sk.encrypt_symmetric(ctx, enc.encode_complex_vector(ctx, z, 2.0 ** 30, chain), seed=22 + n)
        got = ph._apply_layer(ctx, ct, lt, pts, i, bk.glk)
        assert got.chain_index() == chain + 1
        want = _oracle_layer(orc, ph, ctx.N, chain, to_host(ct.data), lt, plan, i, keys)
        assert np.array_equal(to_host(got.data), want), (chain, i)
    assert len(cases) == 6 and rotations >= 12  # babies and giants in both transforms
