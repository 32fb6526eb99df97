"""EvalMod residues on the GPU equal the oracle running the same operation
sequence: the reference's K = 28 family (evalmod_k28_r3: src/evalmod.cu:196-335
Chebyshev basis and weighted sums, :464-605 the K = 28 factoring and double
angles) and this build's degree-63 Chebyshev EvalMod (cheb63), at N = 2^12 and
at the bootstrap's N = 2^16.

Both sides run pyPhantom's EvalMod code unchanged over an engine of ciphertext
operations: the native library's (pyPhantom._GpuEngine) and the CPU oracle's
(tests/oracle_engine.py).  Inputs are uniform residues and a uniform key, so
every limb carries full-range values; the check is residue equality, not
decryption (tests/test_gpu_evalmod.py scores the decrypted values)."""
import numpy as np
import pytest

import py_oracle as O
from gpu_util import to_dev, to_host, uniform_limbs
from oracle_engine import OCt, OracleEngine

pytestmark = pytest.mark.gpu

CASES = {
    # the reference's EvalMod test chain (test/evalmod_test.cu:142-216) at N = 2^12
    "k28_r3": ([58] + [40] * 4 + [58] * 9 + [58], 1, 2.0 ** 58),
    # cheb63 takes 10 levels; 60-bit primes as in bootstrap_coeff_bits, the
    # input at the scale of the first prime its products drop (None below), as
    # in bootstrap (its Chebyshev terms keep that scale)
    "cheb63": ([60] * 12 + [60] * 2, 2, None),
}


def _setup(variant, dev, seed, logN=12):
    import pyPhantom as ph

    N = 1 << logN
    bits, special, scale = CASES[variant]
    mods = ph.create_coeff_modulus(N, bits)
    p = ph.params(ph.scheme_type.ckks)
    p.set_poly_modulus_degree(N)
    p.set_coeff_modulus(mods)
    p.set_special_modulus_size(special)
    ctx = ph.context(p)
    orc = O.Oracle(N, mods, special)
    rng = np.random.default_rng(seed)
    Q = len(mods) - special
    ct_np = uniform_limbs(rng, (2, Q, N), mods)
    key_np = np.stack([uniform_limbs(rng, (2, len(mods), N), mods) for _ in range(orc.dnum)])
    scale = float(mods[Q - 1]) if scale is None else scale
    ct = ph.ciphertext()
    ct.data, ct._chain_index, ct._scale = to_dev(ct_np, dev), 1, scale
    rk = ph.relin_key(to_dev(key_np, dev))
    return ph, ctx, orc, mods, Q, ct, ct_np, rk, key_np, scale


@pytest.mark.parametrize("logN", [12, 16])
@pytest.mark.parametrize("variant", sorted(CASES))
def test_evalmod_residues_match_oracle(dev, variant, logN):
    ph, ctx, orc, mods, Q, ct, ct_np, rk, key_np, scale = _setup(variant, dev, 0xE7A1 + len(variant) + logN, logN)
    gpu = ph._GpuEngine(ctx, rk)
    cpu = OracleEngine(orc, mods, Q, key_np)
    x = OCt(ct_np, 1, scale)
    if variant == "cheb63":
        cheb = ph.evalmod_chebyshev()
        got = ph._eval_mod_cheb(gpu, ct, cheb, ph.BOOT_R)
        want = ph._eval_mod_cheb(cpu, x, cheb, ph.BOOT_R)
    else:
        got = ph._evalmod_ops(gpu, ct, variant)
        want = ph._evalmod_ops(cpu, x, variant)
    assert got.chain_index() == want.chain_index()
    assert got.scale() == want.scale()
    g = to_host(got.data)
    assert g.shape == want.data.shape
    bad = np.argwhere(g != want.data)
    assert bad.size == 0, f"{len(bad)} residues differ, first at {tuple(bad[0])}"
