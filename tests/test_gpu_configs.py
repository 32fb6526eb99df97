"""The benchmark configurations at their full sizes (configs 2-5 of the benchmark,
plus the metric's "L=35" HMult), so that no benchmarked workload is checked
only by bench.py.

* L = 35 HMult + relinearize + rescale (N = 2^16, chain {60, 50 x 34, 60},
  alpha = 1, dnum = 35): multiply_and_relin, rescale and the fused call are
  bit-exact against the oracle's multiply_and_relin_inplace
  (src/evaluate.cu:1061-1104) followed by rescale_to_next (src/rns.cu:1128-1184).
* The key switches of bootstrapping and of the BSGS product at full size
  (N = 2^16, both bootstrappable chains, |Q| = 30 with 6 special primes,
  dnum = 5, top and inner levels; config 4's chain): a rotation and the fused
  HMult + relinearize + rescale bit-exact against the oracle, so the residue
  arithmetic of configs 4 and 5 is pinned at their own shapes, not only at
  N = 2^12.
* Batched HMult (config 3) and batched rotation (config 4 shape) at full size:
  every member equals the single call, which covers the work schedules of the
  batched base-conversion and epilogue launches.
* Config 4, the BSGS matrix-vector product at N = 2^16 (4096 x 4096 matrix
  uniform in [-1/64, 1/64], baby 64 / giant 64, L = 20, scale 2^40): decode
  within 1e-5 of numpy's W x.  The reference's own check of this product is a
  decode tolerance (python/llm_project/blocks/bsgs_test.py:77); its residues are
  pinned bit-exactly at N = 2^12 in test_gpu_bsgs.py.
* Config 5's transforms at full size: the first CoeffToSlot layer and the last
  SlotToCoeff layer bit-exact against the oracle running the same operations.
* Config 5, bootstrapping at N = 2^16 (2^15 slots uniform in [-1, 1], |Q| = 30
  with 6 special primes, dnum = 5, sparse secret h = 192): at least 15 bits of
  refreshed precision (the reference's acceptance bound is 1e-3, about 10 bits,
  test/ckks_engine_test.cu:182-188), and the refreshed ciphertext takes a
  further multiplication.
"""
import math

import numpy as np
import pytest

from gpu_util import empty, first_mismatch, to_dev, to_host
from test_gpu_keyswitch import Setup

pytestmark = pytest.mark.gpu


def test_hmult_L35_alpha1_full_size(dev):
    """The metric's HMult shape: fresh chain-index-1 ciphertexts, 35 digits."""
    st = Setup(16, 35, 1, seed=35)
    assert st.orc.beta(1) == 35 and st.orc.dnum == 35
    a, b = st.ct(1), st.ct(1)
    key = st.key()
    da, db, dk = to_dev(a, dev), to_dev(b, dev), to_dev(key, dev)
    want = st.orc.multiply_and_relin(1, a, b, key, threads=16)
    out = empty((2, 35, st.N), dev)
    st.ctx.multiply_and_relin(1, da, db, dk, out)
    got = to_host(out)
    assert np.array_equal(got, want), first_mismatch(got, want)
    want_r = st.orc.rescale(1, want, threads=16)
    res = empty((2, 34, st.N), dev)
    st.ctx.rescale(1, out, res)
    got = to_host(res)
    assert np.array_equal(got, want_r), first_mismatch(got, want_r)
    fused = empty((2, 34, st.N), dev)
    st.ctx.multiply_relin_rescale(1, da, db, dk, fused)
    got = to_host(fused)
    assert np.array_equal(got, want_r), first_mismatch(got, want_r)


def _full_size_chains():
    """name -> (prime bits, special primes) of the chains configs 4 and 5 run."""
    import pyPhantom as ph

    return {"cheb63": (ph.bootstrap_coeff_bits(), 6), "engine": (ph.ckks_engine_coeff_bits(), 6),
            "config4": ([60] + [40] * 19 + [60] * 4, 4)}


@pytest.mark.parametrize("chain_name,chain", [("cheb63", 1), ("cheb63", 15), ("engine", 1), ("engine", 13),
                                              ("config4", 1)])
def test_keyswitch_bootstrap_chains_full_size(dev, chain_name, chain):
    """The key switches bootstrapping and the BSGS product run, at their full
    size: N = 2^16 over the two bootstrappable chains (|Q| = 30, 6 special
    primes, dnum = 5; 60-, 58- and 50-bit primes in the integer policy next to
    40- and 29-bit ones in the FP64 policy), at the top level (CoeffToSlot's)
    and at a level inside EvalMod / SlotToCoeff, and over config 4's chain
    (|Q| = 20, alpha = 4, dnum = 5).  A rotation (src/evaluate.cu:1607-1656) and
    the fused HMult + relinearize + rescale are bit-exact against the oracle."""
    import pfa_native as P

    bits, alpha = _full_size_chains()[chain_name]
    st = Setup(16, len(bits) - alpha, alpha, seed=50 + chain, bits=bits)
    assert st.orc.dnum == 5
    Ql = st.orc.size_Ql(chain)
    key = st.key()
    dk = to_dev(key, dev)
    ct = st.ct(chain)
    elt = P.galois_elt_from_step(-37, st.N)
    d = to_dev(ct, dev)
    st.ctx.apply_galois(chain, d, elt, dk)
    got, want = to_host(d), st.orc.apply_galois(chain, ct, elt, key, threads=16)
    assert np.array_equal(got, want), first_mismatch(got, want)
    a, b = st.ct(chain), st.ct(chain)
    out = empty((2, Ql - 1, st.N), dev)
    st.ctx.multiply_relin_rescale(chain, to_dev(a, dev), to_dev(b, dev), dk, out)
    want = st.orc.rescale(chain, st.orc.multiply_and_relin(chain, a, b, key, threads=16), threads=16)
    got = to_host(out)
    assert np.array_equal(got, want), first_mismatch(got, want)


@pytest.mark.parametrize("count", [2, 5])
def test_hmult_config3_batch_equals_single_full_size(dev, count):
    """Batched HMult at config 3's full size (N = 2^16, |Q| = 24, alpha = 4):
    every member of pfa_multiply_and_relin_batch and
    pfa_multiply_relin_rescale_batch equals the single call on its pair, bit for
    bit.  At this size the batched base conversion and ModDown epilogue have more
    work items than workgroups and run through their work schedules (position
    -> item tables), which the small-N batch tests of test_gpu_keyswitch.py never
    reach; the single calls are pinned against the oracle at this size there
    (test_multiply_and_relin_config3, test_multiply_relin_rescale_config3)."""
    st = Setup(16, 24, 4, seed=40 + count)
    a = np.stack([st.ct(1) for _ in range(count)])
    b = np.stack([st.ct(1) for _ in range(count)])
    key = st.key()
    da, db, dk = to_dev(a, dev), to_dev(b, dev), to_dev(key, dev)
    single = empty((count, 2, 24, st.N), dev)
    single_r = empty((count, 2, 23, st.N), dev)
    for i in range(count):
        st.ctx.multiply_and_relin(1, da[i], db[i], dk, single[i])
        st.ctx.multiply_relin_rescale(1, da[i], db[i], dk, single_r[i])
    out = empty((count, 2, 24, st.N), dev)
    st.ctx.multiply_and_relin_batch(1, count, da, db, dk, out)
    res = empty((count, 2, 23, st.N), dev)
    st.ctx.multiply_relin_rescale_batch(1, count, da, db, dk, res)
    want, got = to_host(single), to_host(out)
    for i in range(count):
        assert np.array_equal(got[i], want[i]), (i, first_mismatch(got[i], want[i]))
    want, got = to_host(single_r), to_host(res)
    for i in range(count):
        assert np.array_equal(got[i], want[i]), (i, first_mismatch(got[i], want[i]))
    st.ctx.synchronize()


def test_rotate_batch_config4_equals_single_full_size(dev):
    """pfa_rotate_batch at config 4's shape (N = 2^16, chain {60, 40 x 19, 60 x 4},
    alpha = 4; 3 members, each with its own step and key) equals
    pfa_apply_galois on each member, bit for bit: the batched ModUp conversion
    runs through its work schedule here (a single rotation at this shape is
    pinned against the oracle's apply_galois by
    test_keyswitch_bootstrap_chains_full_size)."""
    import pfa_native as P

    st = Setup(16, 20, 4, seed=44, bits=[60] + [40] * 19 + [60] * 4)
    cts = np.stack([st.ct(1) for _ in range(3)])
    keys = [to_dev(st.key(), dev) for _ in range(3)]
    elts = [P.galois_elt_from_step(s, st.N) for s in (64, 1, -3)]
    out = empty(cts.shape, dev)
    st.ctx.rotate_batch(1, to_dev(cts, dev), elts, keys, out)
    got = to_host(out)
    for i in range(3):
        one = to_dev(cts[i], dev)
        st.ctx.apply_galois(1, one, elts[i], keys[i])
        want = to_host(one)
        assert np.array_equal(got[i], want), (i, first_mismatch(got[i], want))
    st.ctx.synchronize()


def test_bsgs_config4_full_size(dev):
    import torch

    import pyPhantom as ph

    N, d_pad, M = 1 << 16, 4096, 64
    p = ph.params(ph.scheme_type.ckks)
    p.set_poly_modulus_degree(N)
    p.set_coeff_modulus(ph.create_coeff_modulus(N, [60] + [40] * 19 + [60] * 4))
    p.set_special_modulus_size(4)
    p.set_galois_elts(ph.get_elts_from_steps(ph.bsgs_required_steps(M), N))
    ctx = ph.context(p)
    sk = ph.secret_key(ctx).generate_sparse(ctx, 192, seed=41)
    glk = sk.create_galois_keys(ctx)
    enc = ph.ckks_encoder(ctx)
    rng = np.random.default_rng(4)
    W = rng.uniform(-1 / 64, 1 / 64, (d_pad, d_pad))
    xv = rng.uniform(-1, 1, d_pad)
    scale = 2.0 ** 40
    diags = ph.pre_encode_bsgs_diagonals(ctx, enc, W.ravel(), d_pad, d_pad, d_pad, M, scale)
    x = sk.encrypt_symmetric(ctx, enc.encode_double_vector(ctx, np.tile(xv, enc.slot_count() // d_pad), scale),
                             seed=42)
    y = ph.bsgs_matmul_preencoded(ctx, glk, x, diags)
    got = np.array(enc.decode_double_vector(ctx, sk.decrypt(ctx, y)))
    want = np.tile(W @ xv, enc.slot_count() // d_pad)
    err = float(np.max(np.abs(got - want)))
    print(f"config 4 BSGS: max |err| {err:.3e}")
    assert y.chain_index() == x.chain_index() + 1
    assert err < 1e-5
    del diags, glk
    torch.cuda.empty_cache()


@pytest.fixture(scope="module")
def boot16(dev):
    import pyPhantom as ph

    N = 1 << 16
    p = ph.params(ph.scheme_type.ckks)
    p.set_poly_modulus_degree(N)
    p.set_coeff_modulus(ph.create_coeff_modulus(N, ph.bootstrap_coeff_bits()))
    p.set_special_modulus_size(6)
    p.set_galois_elts(ph.bootstrap_required_galois_elts(16))
    ctx = ph.context(p)
    assert ctx.size_Q == 30 and ctx.size_P == 6
    sk = ph.secret_key(ctx).generate_sparse(ctx, 192, seed=51)
    enc = ph.ckks_encoder(ctx)
    bk = ph.create_bootstrap_key(ctx, enc, sk, sparse_hamming_weight=192, seed=52, evalmod="cheb63")
    yield ph, ctx, sk, enc, bk
    import torch

    del bk
    torch.cuda.empty_cache()


@pytest.mark.parametrize("which", ["c2s_first", "s2c_last"])
def test_bootstrap_transform_layer_full_size(boot16, which):
    """One CoeffToSlot layer (the first, at the top of the chain) and one
    SlotToCoeff layer (the last) at config 5's size, as bootstrap runs them
    (hoisted babies, pfa_bsgs_mac, the batched giants, the sum, the rescale),
    bit-exact against the oracle running the same operations one by one: the
    residue pin of the transforms at N = 2^16 (all six layers are pinned at
    N = 2^12 in test_gpu_bootstrap.py)."""
    import py_oracle as O
    from test_gpu_bootstrap import _oracle_layer

    ph, ctx, sk, enc, bk = boot16
    if which == "c2s_first":
        lt, pts, i, chain = bk.c2s, bk.c2s_pts, 0, 1
    else:
        lt, pts, i = bk.s2c, bk.s2c_pts, len(bk.s2c_pts) - 1
        chain = bk.s2c_start + i
    plan = pts[i]
    rng = np.random.default_rng(60 + i)
    z = rng.uniform(-1, 1, enc.slot_count()) + 1j * rng.uniform(-1, 1, enc.slot_count())
    ct = sk.encrypt_symmetric(ctx, enc.encode_complex_vector(ctx, z, 2.0 ** 40, chain), seed=61)
    got = ph._apply_layer(ctx, ct, lt, pts, i, bk.glk)
    assert got.chain_index() == chain + 1
    orc = O.Oracle(ctx.N, ctx.moduli, ctx.size_P)
    # only the layer's own keys come to the host (one is up to 180 MB here)
    n1, unit = lt.baby_giant(i)[0], lt.units[i]
    used = {ph.get_elt_from_step(b * unit, ctx.N) for b in plan.babies if b}
    used |= {ph.get_elt_from_step(ph._signed_step(g * n1 * unit, lt.n), ctx.N) for g in plan.giants if g}
    keys = {e: to_host(bk.glk.keys[e]) for e in used}
    want = _oracle_layer(orc, ph, ctx.N, chain, to_host(ct.data), lt, plan, i, keys)
    got = to_host(got.data)
    assert np.array_equal(got, want), first_mismatch(got, want)


def test_bootstrap_config5_full_size(boot16):
    ph, ctx, sk, enc, bk = boot16
    n = enc.slot_count()
    assert n == 1 << 15
    z = np.random.default_rng(5).uniform(-1, 1, n)
    scale = 2.0 ** 40
    ct = sk.encrypt_symmetric(ctx, enc.encode_double_vector(ctx, z, scale, ctx.size_Q), seed=53)
    out = ph.bootstrap(ctx, enc, ct, bk, scale)
    got = np.array(enc.decode_double_vector(ctx, sk.decrypt(ctx, out)))
    err = float(np.max(np.abs(got - z)))
    bits = -math.log2(err)
    print(f"config 5 bootstrap: max |err| {err:.3e} ({bits:.2f} bits), chain index {out.chain_index()}")
    assert bits >= 15
    # a further multiplication on the refreshed ciphertext decodes to z^2
    sq = ph.rescale_to_next(ctx, ph.multiply_and_relin(ctx, out, out, bk.rlk))
    got2 = np.array(enc.decode_double_vector(ctx, sk.decrypt(ctx, sq)))
    assert np.max(np.abs(got2 - z * z)) < 1e-4


@pytest.fixture(scope="module")
def engine16(dev):
    import pyPhantom as ph

    N = 1 << 16
    p = ph.params(ph.scheme_type.ckks)
    p.set_poly_modulus_degree(N)
    p.set_coeff_modulus(ph.create_coeff_modulus(N, ph.ckks_engine_coeff_bits()))
    p.set_special_modulus_size(6)
    p.set_galois_elts(ph.bootstrap_required_galois_elts(16))
    ctx = ph.context(p)
    assert ctx.size_Q == 30 and ctx.size_P == 6
    sk = ph.secret_key(ctx).generate_sparse(ctx, 192, seed=81)
    enc = ph.ckks_encoder(ctx)
    bk = ph.create_bootstrap_key(ctx, enc, sk, sparse_hamming_weight=192, eval_mod_levels=9,
                                 user_scale=2.0 ** 40, seed=82)
    yield ph, ctx, sk, enc, bk
    import torch

    del bk
    torch.cuda.empty_cache()


def test_bootstrap_config5_evalround(engine16):
    """Config 5 through the reference's pipeline: the engine's chain
    (q_msg 58 | 14 x 40 | 3 x 58 | 9 x 58 | 3 x 29 + 6 x 58 special, |Q| = 30,
    dnum = 5), EvalRound with evalmod_k28_r3, SlotToCoeff at user scale 2^40,
    the ciphertext entering one level above the bottom as the engine
    hands it over; the reference's bar is 1e-3 (test/ckks_engine_test.cu:182)."""
    ph, ctx, sk, enc, bk = engine16
    n = enc.slot_count()
    z = np.random.default_rng(5).uniform(-1, 1, n)
    scale = 2.0 ** 40
    ct = sk.encrypt_symmetric(ctx, enc.encode_double_vector(ctx, z, scale, ctx.size_Q - 1), seed=83)
    out = ph.bootstrap(ctx, enc, ct, bk, scale)
    assert out.chain_index() == 16 and abs(out.scale() / scale - 1) < 1e-9
    got = np.array(enc.decode_double_vector(ctx, sk.decrypt(ctx, out)))
    err = float(np.max(np.abs(got - z)))
    bits = -math.log2(err)
    print(f"config 5 EvalRound bootstrap: max |err| {err:.3e} ({bits:.2f} bits)")
    assert err < 1e-3
    sq = ph.rescale_to_next(ctx, ph.multiply_and_relin(ctx, out, out, bk.rlk))
    got2 = np.array(enc.decode_double_vector(ctx, sk.decrypt(ctx, sq)))
    assert np.max(np.abs(got2 - z * z)) < 4e-3
