"""inner_sum / replicate (src/linear.cu) and eval_polynomial (src/ps.cu):
decoded results against numpy, the levels each consumes, the reference's
argument errors, and residues equal to the same sequence of evaluator calls
composed by hand (inner_sum)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

N = 1 << 13


@pytest.fixture(scope="module")
def env():
    import pyPhantom as ph

    p = ph.params(ph.scheme_type.ckks)
    p.set_poly_modulus_degree(N)
    p.set_coeff_modulus(ph.create_coeff_modulus(N, [60] + [40] * 11 + [60, 60]))  # |Q| = 12, dnum = 6
    p.set_special_modulus_size(2)
    steps = [1, 2, 4, 8, -8, -16, -32, -64]
    p.set_galois_elts(ph.get_elts_from_steps(steps, N))
    ctx = ph.context(p)
    sk = ph.secret_key(ctx, seed=11).generate_sparse(ctx, 192)
    return ph, ctx, sk, sk.gen_relinkey(ctx, seed=12), sk.create_galois_keys(ctx, seed=13), ph.ckks_encoder(ctx)


def _dec(env, ct):
    ph, ctx, sk, _, _, enc = env
    return np.array(enc.decode_double_vector(ctx, sk.decrypt(ctx, ct)))


def test_inner_sum(env):
    ph, ctx, sk, _, glk, enc = env
    v = np.random.default_rng(1).uniform(-1, 1, N // 2)
    ct = sk.encrypt_symmetric(ctx, enc.encode_double_vector(ctx, v, 2.0 ** 40), seed=2)
    out = ph.inner_sum(ctx, glk, ct, 16)
    got = _dec(env, out)
    want = v.reshape(-1, 16).sum(axis=1)
    assert np.max(np.abs(got[::16] - want)) < 1e-5
    # the same residues as the rotate-and-add sequence
    acc = ct
    for s in (1, 2, 4, 8):
        acc = ph.add(ctx, acc, ph.rotate(ctx, acc, s, glk))
    assert np.array_equal(out.data.cpu().numpy(), acc.data.cpu().numpy())
    assert out.chain_index() == ct.chain_index()
    with pytest.raises(ValueError):
        ph.inner_sum(ctx, glk, ct, 12)


def test_replicate(env):
    ph, ctx, sk, _, glk, enc = env
    v = np.zeros(N // 2)
    v[:8] = np.random.default_rng(3).uniform(-1, 1, 8)
    ct = sk.encrypt_symmetric(ctx, enc.encode_double_vector(ctx, v, 2.0 ** 40), seed=4)
    got = _dec(env, ph.replicate(ctx, glk, ct, 8, 128))
    assert np.max(np.abs(got[:128] - np.tile(v[:8], 16))) < 1e-5
    for args in ((6, 128), (8, 96), (256, 128)):
        with pytest.raises(ValueError):
            ph.replicate(ctx, glk, ct, *args)


@pytest.mark.parametrize("coeffs", [[0.25, -0.5], [0.1, 0.2, -0.3], [0.1, -0.5, 0.3, 0.2, -0.1, 0.05, 0.02, -0.01],
                                    [0.0, 1.0, 0.0, -1 / 6, 0.0, 1 / 120, 0.0, -1 / 5040, 0.0, 1 / 362880]])
def test_eval_polynomial(env, coeffs):
    ph, ctx, sk, rlk, _, enc = env
    x = np.random.default_rng(5).uniform(-1, 1, N // 2)
    ct = sk.encrypt_symmetric(ctx, enc.encode_double_vector(ctx, x, 2.0 ** 40), seed=6)
    out = ph.eval_polynomial(ctx, enc, rlk, ct, coeffs)
    d = len(coeffs) - 1
    m = int(np.ceil(np.sqrt(d + 1)))
    l = (d + 1 + m - 1) // m
    assert out.chain_index() == ct.chain_index() + m + l - 2
    assert out.scale() == ct.scale()
    want = np.polyval(coeffs[::-1], x)
    assert np.max(np.abs(_dec(env, out) - want)) < 1e-5
    with pytest.raises(ValueError):
        ph.eval_polynomial(ctx, enc, rlk, ct, [1.0])
