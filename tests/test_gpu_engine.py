"""ckks_engine, the reference's bootstrappable facade (src/ckks_engine.cu,
python/src/binding.cu:339-382), at its one size (log_n = 16).

* The three cases of the reference's own engine test (test/ckks_engine_test.cu)
  with its tolerances: encode / encrypt / decrypt within 1e-7, multiply +
  relinearize + rescale within 1e-5 at user level 1, and a ciphertext depleted
  to max_user_level() by plaintext multiplies and rescales, bootstrapped back to
  user level 0 within 1e-3.
* The user rotations (+-1, +-2 by default) through galois_key(); a step that
  CoeffToSlot / SlotToCoeff also use shares the bootstrap key's tensor.
* split_scale_down: the bootstrap returns at user level 1.
* use_bootstrap_to_17_levels: its chain, round trips, a refused bootstrap, and
  the per-level scale arrays (build_two_scale_arrays) against the recurrence's
  defining properties.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def engine():
    import pyPhantom as ph

    return ph.ckks_engine(ph.ckks_engine_config(), seed=7)


def _max_err(got, want):
    return float(np.max(np.abs(np.asarray(got) - np.asarray(want))))


def test_engine_layout(engine):
    import pyPhantom as ph

    ctx = engine.context()
    bits = [q.bit_length() for q in ctx.moduli]
    assert bits == ph.ckks_engine_coeff_bits(14, 6)
    assert engine.slot_count() == 1 << 15 and engine.user_scale() == 2.0 ** 40
    assert engine.max_user_level() == 13
    # user level k at chain 16 + k (3 CoeffToSlot + 9 EvalRound + 3 SlotToCoeff above it)
    assert [engine.user_level_chain_index(k) for k in (0, 13)] == [16, 29]
    with pytest.raises(ValueError):
        engine.user_level_chain_index(14)
    assert engine.scale_array_size() == 0 and engine.ckks_scale_at(0) == 0.0


def test_engine_round_trip(engine):
    rng = np.random.default_rng(0xCAFE)
    z = rng.uniform(-0.5, 0.5, engine.slot_count()) + 1j * rng.uniform(-0.5, 0.5, engine.slot_count())
    ct = engine.encrypt(engine.encode(z))
    assert engine.user_level(ct) == 0
    assert _max_err(engine.decrypt_decode(ct), z) < 1e-7


def test_engine_mul_and_rescale(engine):
    rng = np.random.default_rng(0xBABE)
    a, b = rng.uniform(-0.5, 0.5, engine.slot_count()), rng.uniform(-0.5, 0.5, engine.slot_count())
    ca, cb = engine.encrypt(engine.encode(a, 0)), engine.encrypt(engine.encode(b, 0))
    engine.mul_and_relin_inplace(ca, cb)
    engine.rescale_inplace(ca)
    assert engine.user_level(ca) == 1
    assert _max_err(engine.decrypt_decode(ca), a * b) < 1e-5


def test_engine_deplete_then_bootstrap(engine):
    rng = np.random.default_rng(0xB00B007)
    n = engine.slot_count()
    x = rng.uniform(-0.5, 0.5, n)
    ct = engine.encrypt(engine.encode(x, 0))
    ones = np.ones(n)
    for k in range(engine.max_user_level()):
        engine.mul_plain_inplace(ct, engine.encode(ones, k))
        engine.rescale_inplace(ct)
    assert engine.user_level(ct) == engine.max_user_level()
    with pytest.raises(RuntimeError):  # the next level is the bootstrap's own
        engine.rescale_inplace(ct)
    engine.bootstrap_inplace(ct)
    assert engine.user_level(ct) == 0 and ct.scale() == engine.user_scale()
    err = float(np.max(np.abs(np.real(engine.decrypt_decode(ct)) - x)))
    assert err < 1e-3, err
    # a bootstrapped ciphertext takes a further multiplication
    engine.mul_and_relin_inplace(ct, engine.encrypt(engine.encode(x, 0)))
    engine.rescale_inplace(ct)
    assert _max_err(np.real(engine.decrypt_decode(ct)), x * x) < 1e-3


def test_engine_user_rotations(engine):
    """Rotations of a fresh ciphertext at user_scale 2^40.  Slot 0 carries the
    key switch's offset term of the reference's algorithm: its ModDown
    conversion (uncorrected, src/rns_bconv.cu:212-229) leaves a non-negative
    integer in [0, alpha) on every coefficient, and that offset's mean
    (alpha - 1) / 2 times the engine's dense secret is a low-frequency error of
    about ((alpha - 1) / 2) (2N / pi) |s(zeta)| / scale ~ 2.5 x 41722 x 209 / 2^40
    ~ 2e-5 in slot 0, falling as 1 / 5^j in slot j (measured 4.4e-5, 8e-6,
    5e-7 for every step and key; a fresh ciphertext decodes within 2.4e-9).
    So the bound is 2e-4 on the worst slot and 1e-7 on the median."""
    import pyPhantom as ph

    n = engine.slot_count()
    z = np.random.default_rng(3).uniform(-0.5, 0.5, n)
    ct = engine.encrypt(engine.encode(z, 0))
    glk, boot = engine.galois_key(), engine.bootstrap_key().glk
    boot_steps = set(ph.c2s_required_rotation_steps(ph.build_c2s_diagonals(16), n)) | \
        set(ph.c2s_required_rotation_steps(ph.build_s2c_diagonals(16), n))
    for step in (1, -1, 2, -2):
        elt = ph.get_elt_from_step(step, 2 * n)
        assert (glk.keys[elt] is boot.keys.get(elt)) == (step in boot_steps)
        r = ph.ciphertext()
        r.data, r._chain_index, r._scale = ct.data.clone(), ct.chain_index(), ct.scale()
        engine.rotate_inplace(r, step)
        e = np.abs(np.real(engine.decrypt_decode(r)) - np.roll(z, -step))
        assert e.max() < 2e-4 and np.median(e) < 1e-7, (step, e.max(), np.median(e))
    # conjugation: the user bundle's key, which the bootstrap also reads
    conj = 4 * n - 1
    assert glk.keys[conj] is boot.keys[conj]


def test_engine_split_scale_down():
    import pyPhantom as ph

    cfg = ph.ckks_engine_config()
    cfg.split_scale_down = True
    cfg.include_user_rotations = False
    eng = ph.ckks_engine(cfg, seed=8)
    x = np.random.default_rng(4).uniform(-0.5, 0.5, eng.slot_count())
    ct = eng.encrypt(eng.encode(x, eng.max_user_level()))
    eng.bootstrap_inplace(ct)
    assert eng.user_level(ct) == 1
    err = float(np.max(np.abs(np.real(eng.decrypt_decode(ct)) - x)))
    assert err < 1e-3, err
    conj = 2 * (1 << 16) - 1
    assert set(eng.galois_key().keys) == {conj}


def test_engine_bootstrap_to_17_levels_chain_and_scales():
    import pyPhantom as ph

    cfg = ph.ckks_engine_config()
    cfg.use_bootstrap_to_17_levels = True
    cfg.num_scale_levels = 16  # 16 + 14 = 30 primes, divisible by 6
    cfg.build_two_scale_arrays = True
    eng = ph.ckks_engine(cfg, seed=9)
    ctx = eng.context()
    assert [q.bit_length() for q in ctx.moduli] == [40] * 16 + [29] + [54] * 12 + [42] + [60] * 6
    assert eng.user_level_chain_index(0) == 14 and eng.max_user_level() == 15
    z = np.random.default_rng(5).uniform(-0.5, 0.5, eng.slot_count())
    ct = eng.encrypt(eng.encode(z, 0))
    assert eng.user_level(ct) == 0
    assert _max_err(np.real(eng.decrypt_decode(ct)), z) < 1e-6
    with pytest.raises(RuntimeError):
        eng.bootstrap_inplace(ct)
    # scale arrays: ckks_scale[0] = user_scale^2; each rescaled entry is the
    # squared one over the last prime of that chain index (the key level's
    # last prime is the last special one), and the next squared entry is its
    # square; past the end, 0
    T = ctx.total_parm_size()
    assert eng.scale_array_size() == T and eng.ckks_scale_at(T) == 0.0
    assert eng.ckks_scale_at(0) == 2.0 ** 80
    for i in range(T):
        last = ctx.moduli[-1] if i == 0 else ctx.moduli[ctx.size_Ql(i) - 1]
        s, r = eng.ckks_scale_at(i), eng.ckks_rescaled_scale_at(i)
        if s > 1e-290:
            assert r == pytest.approx(s / last, rel=4e-16), i
        if i + 1 < T and r > 1e-140:
            assert eng.ckks_scale_at(i + 1) == pytest.approx(r * r, rel=4e-16), i
