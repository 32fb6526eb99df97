"""GPU tests of the reference's EvalMod family and its EvalRound bootstrap.

* evalmod_k7_r3 / evalmod_k16_r3 / evalmod_k28_r3 (src/evalmod.cu) on the
  reference's own test setup (test/evalmod_test.cu:142-216,
  run_lapis_4section): N = 2^16, chain q_msg 58 | 40 x 4 | 58 x 9 | special 58,
  sparse secret of weight 128, inputs uniform in [-0.5, 0.5] encoded at 2^58,
  every slot scored against sin(2 pi K x) / (2 pi) with the reference's
  tolerances (5e-7 for K = 16 and 28, 5e-5 for K = 7), and against the float64
  model of the same polynomial (tests/test_bootstrap_math.py pins the model
  against the sine).
* The reference's bootstrap pipeline (create_bootstrap_key with
  eval_mod_levels = 9: EvalRound K = 28, saved - SlotToCoeff(round)) at
  N = 2^12 on the engine's chain layout (ckks_engine_coeff_bits), baked and
  split scale-down, within the reference's 1e-3 acceptance bar
  (test/ckks_engine_test.cu:182); the round-trip key (eval_mod_levels = 0:
  CoeffToSlot then SlotToCoeff) returns the input and is refused by
  bootstrap(), as in the reference.
"""
import math

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lapis16(dev):
    import pyPhantom as ph

    N = 1 << 16
    p = ph.params(ph.scheme_type.ckks)
    p.set_poly_modulus_degree(N)
    p.set_coeff_modulus(ph.create_coeff_modulus(N, [58] + [40] * 4 + [58] * 9 + [58]))
    p.set_special_modulus_size(1)
    ctx = ph.context(p)
    sk = ph.secret_key().generate_sparse(ctx, 128, seed=61)
    rk = sk.gen_relinkey(ctx, seed=62)
    enc = ph.ckks_encoder(ctx)
    yield ph, ctx, sk, rk, enc
    import torch

    del rk
    torch.cuda.empty_cache()


@pytest.mark.parametrize("variant,tol", [("k28_r3", 5e-7), ("k16_r3", 5e-7), ("k7_r3", 5e-5)])
def test_evalmod_reference_setup(lapis16, variant, tol):
    ph, ctx, sk, rk, enc = lapis16
    K = ph.EVALMOD_K[variant]
    x = np.random.default_rng(0xC0FFEE ^ K).uniform(-0.5, 0.5, enc.slot_count())
    ct = sk.encrypt_symmetric(ctx, enc.encode_double_vector(ctx, x, 2.0 ** 58, 1), seed=63)
    out = getattr(ph, "evalmod_" + variant)(ctx, enc, ct, rk)
    assert out.chain_index() == 1 + ph.EVALMOD_LEVELS[variant]
    assert out.scale() == ct.scale()  # snapped back to the input scale, as in the reference
    got = np.array(enc.decode_double_vector(ctx, sk.decrypt(ctx, out)))
    err_sin = float(np.max(np.abs(got - np.sin(2 * np.pi * K * x) / (2 * np.pi))))
    err_model = float(np.max(np.abs(got - ph.evalmod_model(x, variant))))
    print(f"evalmod_{variant}: max |err| vs sine {err_sin:.3e}, vs model {err_model:.3e}")
    assert err_sin < tol
    assert err_model < tol


def test_evalmod_needs_its_levels(lapis16):
    ph, ctx, sk, rk, enc = lapis16
    x = np.zeros(enc.slot_count())
    ct = sk.encrypt_symmetric(ctx, enc.encode_double_vector(ctx, x, 2.0 ** 58, 6), seed=64)
    with pytest.raises(ValueError):
        ph.evalmod_k28_r3(ctx, enc, ct, rk)


def engine_setup(logN=12, nsl=2, special=3, hw=128, seed=70):
    import pyPhantom as ph

    N = 1 << logN
    stages = ph._default_stages(logN)
    p = ph.params(ph.scheme_type.ckks)
    p.set_poly_modulus_degree(N)
    p.set_coeff_modulus(ph.create_coeff_modulus(N, ph.ckks_engine_coeff_bits(nsl, special)))
    p.set_special_modulus_size(special)
    p.set_galois_elts(ph.bootstrap_required_galois_elts(logN, stages))
    ctx = ph.context(p)
    sk = ph.secret_key(ctx, seed=seed)
    enc = ph.ckks_encoder(ctx)
    return ph, ctx, sk, enc


@pytest.fixture(scope="module")
def engine12(dev):
    return engine_setup()


@pytest.mark.parametrize("split", [False, True])
def test_bootstrap_evalround(engine12, split):
    """The pipeline's own error is EvalRound's (2 pi)^2 eps^3 / 6 per coefficient,
    eps = the message's coefficient over the scale q_msg it is lifted to, about
    |z| / sqrt(N): ~8e-3 in the slots at N = 2^12 for |z| <= 1 (1e-4 rms at
    N = 2^16, the size the reference runs it at).  So the mechanics are checked
    here on a message of 1/16 the size (error 16^3 smaller), and the full-range
    message against the cubic estimate."""
    ph, ctx, sk, enc = engine12
    user_scale = 2.0 ** 40
    bk = ph.create_bootstrap_key(ctx, enc, sk, 128, eval_mod_levels=9, user_scale=user_scale,
                                 split_scale_down=split, seed=71)
    assert bk.evalmod == "k28_r3"
    n = enc.slot_count()
    rng = np.random.default_rng(72)
    z = rng.uniform(-1, 1, n) + 1j * rng.uniform(-1, 1, n)
    for amp, bar in ((1 / 16, 1e-4), (1.0, 2e-2)):
        ct = sk.encrypt_symmetric(ctx, enc.encode_complex_vector(ctx, amp * z, user_scale, ctx.size_Q - 1), seed=73)
        out = ph.bootstrap(ctx, enc, ct, bk, user_scale, split)
        assert out.chain_index() == 1 + 3 + 9 + 3 + (1 if split else 0)
        # split: snapped to user_scale; baked: user_scale times the ratio of the
        # primes SlotToCoeff's first and last layers drop (src/bootstrap.cu:1801-1803)
        assert out.scale() == user_scale if split else abs(out.scale() / user_scale - 1) < 1e-9
        got = np.array(enc.decode_complex_vector(ctx, sk.decrypt(ctx, out)))
        err = float(np.max(np.abs(got - amp * z)))
        print(f"EvalRound bootstrap N=2^12 split={split} |z|<={amp}: max |err| {err:.3e} ({-math.log2(err):.1f} bits)")
        assert err < bar
    sq = ph.rescale_to_next(ctx, ph.multiply_and_relin(ctx, out, out, bk.rlk))
    got2 = np.array(enc.decode_complex_vector(ctx, sk.decrypt(ctx, sq)))
    assert np.max(np.abs(got2 - z * z)) < 4e-2
    with pytest.raises(ValueError):
        ph.bootstrap(ctx, enc, ct, bk, user_scale, not split)


def test_round_trip_key(engine12):
    """eval_mod_levels = 0: CoeffToSlot chained straight into SlotToCoeff returns
    the slots (src/bootstrap.cu:936-958); bootstrap() refuses the key."""
    ph, ctx, sk, enc = engine12
    bk = ph.create_bootstrap_key(ctx, enc, sk, 128, seed=74)
    assert bk.eval_mod_levels == 0
    n = enc.slot_count()
    rng = np.random.default_rng(75)
    z = rng.uniform(-1, 1, n) + 1j * rng.uniform(-1, 1, n)
    ct = sk.encrypt_symmetric(ctx, enc.encode_complex_vector(ctx, z, 2.0 ** 58, 1), seed=76)
    rt = ph.apply_s2c_inplace(ctx, ph.apply_c2s_inplace(ctx, ct, bk), bk)
    assert rt.chain_index() == 1 + 6
    got = np.array(enc.decode_complex_vector(ctx, sk.decrypt(ctx, rt)))
    err = float(np.max(np.abs(got - z)))
    print(f"C2S -> S2C round trip: max |err| {err:.3e}")
    assert err < 1e-3  # the reference's round-trip bar (test/bootstrap_test.cu:313)
    with pytest.raises(RuntimeError):
        ph.bootstrap(ctx, enc, ct, bk, 2.0 ** 58)


def test_bootstrap_key_arguments(engine12):
    ph, ctx, sk, enc = engine12
    with pytest.raises(ValueError):
        ph.create_bootstrap_key(ctx, enc, sk, 128, eval_mod_levels=9, evalmod="cheb63")
    with pytest.raises(ValueError):
        ph.create_bootstrap_key(ctx, enc, sk, 128, user_scale=2.0 ** 40, evalmod="cheb63")
    with pytest.raises(ValueError):
        ph.create_bootstrap_key(ctx, enc, sk, 128, evalmod="k99")
    with pytest.raises(ValueError):
        ph.create_bootstrap_key(ctx, enc, sk, 128, eval_mod_levels=40)


def test_evalmod_bundle_matches_tracks(lapis16):
    """Bootstrap runs EvalMod on its real and imaginary tracks as one bundle
    (each step one batched native call): the bundle's members are bit-identical
    to EvalMod of each ciphertext alone, with the same level and scale."""
    ph, ctx, sk, rk, enc = lapis16
    rng = np.random.default_rng(71)
    cts = [sk.encrypt_symmetric(ctx, enc.encode_double_vector(ctx, rng.uniform(-0.5, 0.5, enc.slot_count()),
                                                              2.0 ** 58, 1), seed=72 + i) for i in range(2)]
    alone = [ph.evalmod_k28_r3(ctx, enc, c, rk) for c in cts]
    both = ph._unbundle(ph._evalmod(ctx, ph._bundle(ctx, cts), rk, "k28_r3"))
    for a, b in zip(alone, both):
        assert a.chain_index() == b.chain_index() and a.scale() == b.scale()
        assert bool((a.data == b.data).all())
