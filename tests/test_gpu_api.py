"""GPU tests of the pyPhantom drop-in module, the CKKS encoder and hoisting.

* hoisting (pfa_hoisting) is bit-exact against the oracle, whose restatement of
  src/evaluate.cu:1732-1927 is pinned in tests/test_oracle.py.
* The encoder (pfa_ckks_encode/decode) is checked against a numpy statement of
  the canonical embedding (slot j = m(zeta^(5^j)), evaluated directly at small N)
  and by round trips.  The reference's special FFT cannot run here (CUDA only),
  so the plaintext bit pattern is "parity unpinned"; decoded slots are held to
  the north star's 1e-6 absolute tolerance.
* The end-to-end flow mirrors the reference's python/examples/ckks.py and
  examples/3_ckks.cu (decrypt-decode within a tolerance after mul + relin +
  rescale, rotation and hoisting).
"""
import numpy as np
import pytest

import py_oracle as O
from gpu_util import empty, first_mismatch, to_dev, to_host, uniform_limbs

pytestmark = pytest.mark.gpu

TOL = 1e-6


def make_ctx(logN, bits, special, steps=()):
    import pyPhantom as ph

    N = 1 << logN
    p = ph.params(ph.scheme_type.ckks)
    p.set_poly_modulus_degree(N)
    p.set_coeff_modulus(ph.create_coeff_modulus(N, bits))
    p.set_special_modulus_size(special)
    p.set_galois_elts(ph.get_elts_from_steps(list(steps), N))
    return ph, ph.context(p)


# ----------------------------------------------------------------- hoisting
@pytest.mark.parametrize("logN,nq,alpha,chain", [(12, 6, 2, 1), (12, 5, 1, 2), (16, 6, 3, 1)])
def test_hoisting_matches_oracle(dev, logN, nq, alpha, chain):
    import pfa_native as P

    N = 1 << logN
    mods = O.create_coeff_modulus(N, [60] + [50] * (nq - 1) + [60] * alpha)
    ctx = P.NativeContext(N, mods, alpha)
    orc = O.Oracle(N, mods, alpha)
    rng = np.random.default_rng(logN + nq)
    Ql = orc.size_Ql(chain)
    ct = uniform_limbs(rng, (2, Ql, N), mods)
    steps = [1, 3, -2]
    elts = [P.galois_elt_from_step(s, N) for s in steps]
    keys = [uniform_limbs(rng, (orc.dnum, 2, len(mods), N), mods) for _ in steps]
    out = empty((2, Ql, N), dev)
    ctx.hoisting(chain, to_dev(ct, dev), elts, [to_dev(k, dev) for k in keys], out)
    got, want = to_host(out), orc.hoisting(chain, ct, elts, keys, threads=8)
    assert np.array_equal(got, want), first_mismatch(got, want)


# ----------------------------------------------------------------- encoder
def embed_direct(coeffs, n):
    """slot_j = sum_k m_k zeta^(k 5^j), zeta = exp(2 pi i / 2n), j < n/2."""
    m2 = 2 * n
    ks = np.arange(n)
    exps = np.array([pow(5, j, m2) for j in range(n // 2)])
    return np.exp(2j * np.pi * (np.outer(exps, ks) % m2) / m2) @ coeffs


def test_encoder_matches_direct_embedding(dev):
    """Decode of a known integer plaintext = the canonical embedding evaluated directly."""
    import torch

    ph, ctx = make_ctx(11, [60, 50, 50, 60], 1)
    n = ctx.N
    rng = np.random.default_rng(1)
    coeffs = rng.integers(-(2 ** 40), 2 ** 40, n).astype(np.int64)
    L = ctx.size_Ql(1)
    pt = ctx._signed_to_rns(coeffs, L)
    ctx.native.ntt_forward(pt, 1, L, 0)
    out = torch.empty(n // 2, dtype=torch.complex128, device=dev)
    ctx.native.ckks_decode(pt, L, 1.0, out)
    got = out.cpu().numpy()
    want = embed_direct(coeffs.astype(np.float64), n)
    assert np.max(np.abs(got - want)) / 2 ** 40 < 1e-9


def test_encoder_encode_is_inverse_embedding(dev):
    """Encode rounds scale * (inverse embedding); re-embedding the integer
    coefficients gives back the values to within rounding (|err| < n / scale)."""
    import torch

    ph, ctx = make_ctx(11, [60, 50, 50, 60], 1)
    n = ctx.N
    rng = np.random.default_rng(2)
    vals = rng.uniform(-1, 1, n // 2) + 1j * rng.uniform(-1, 1, n // 2)
    scale = 2.0 ** 30
    L = ctx.size_Ql(1)
    pt = empty((L, n), dev)
    ctx.native.ckks_encode(torch.from_numpy(vals).to(dev), scale, pt, L)
    coef = O.Oracle(n, ctx.moduli, 1).ntt_inv(to_host(pt))[0].astype(np.int64)
    q0 = ctx.moduli[0]
    coef = np.where(coef > q0 // 2, coef - q0, coef).astype(np.float64)
    back = embed_direct(coef, n) / scale
    assert np.max(np.abs(back - vals)) < n / scale


@pytest.mark.parametrize("logN,chain", [(12, 1), (16, 1), (16, 3)])
def test_encode_decode_roundtrip(dev, logN, chain):
    ph, ctx = make_ctx(logN, [60, 40, 40, 40, 60], 1)
    enc = ph.ckks_encoder(ctx)
    rng = np.random.default_rng(logN)
    vals = rng.uniform(-1, 1, enc.slot_count())
    pt = enc.encode_double_vector(ctx, vals, 2.0 ** 40, chain_index=chain)
    dec = np.array(enc.decode_double_vector(ctx, pt))
    assert np.max(np.abs(dec - vals)) < 1e-9
    cv = vals[:100] + 1j * vals[100:200]
    pc = enc.encode_complex_vector(ctx, cv, 2.0 ** 40, chain_index=chain)
    dc = np.array(enc.decode_complex_vector(ctx, pc))
    assert np.max(np.abs(dc[:100] - cv)) < 1e-9 and np.max(np.abs(dc[100:])) < 1e-9


def _crt_centred(res, mods):
    """Residues [L][N] -> the centred integers they represent (Python ints)."""
    Q = 1
    for q in mods:
        Q *= q
    out = []
    for k in range(res.shape[1]):
        x = 0
        for l, q in enumerate(mods):
            Ql = Q // q
            x += int(res[l, k]) * Ql * pow(Ql, -1, q)
        x %= Q
        out.append(x - Q if x > (Q - 1) // 2 else x)
    return out


def test_encoder_large_coefficients_exact(dev):
    """Scale 2^125 over four primes (210 bits): coefficients near 2^119 are
    reduced into every prime exactly (the reference's multi-word decomposition,
    src/rns_base.cu:75-170), so the residues CRT-compose to integers whose
    embedding is the input; decoding composes all four limbs (compose_array,
    src/rns_base.cu:173-253), beyond q0 q1 / 2 ~ 2^109 where two limbs stop
    being enough.  The single-chain coefficients at the same scale are those
    integers reduced mod q0 and centred (src/single_chain_plaintext.cu:93-150)."""
    import torch

    ph, ctx = make_ctx(12, [60, 50, 50, 50, 60], 1)
    n, L, scale = ctx.N, ctx.size_Ql(1), 2.0 ** 125
    rng = np.random.default_rng(125)
    vals = rng.uniform(-1, 1, n // 2) + 1j * rng.uniform(-1, 1, n // 2)
    pt = empty((L, n), dev)
    dv = torch.from_numpy(vals).to(dev)
    ctx.native.ckks_encode(dv, scale, pt, L)
    mods = list(ctx.moduli[:L])
    X = _crt_centred(O.Oracle(n, ctx.moduli, 1).ntt_inv(to_host(pt)), mods)
    assert max(abs(x) for x in X) > 1 << 112  # beyond two 50/60-bit limbs
    back = embed_direct(np.array([float(x) / scale for x in X]), n)
    assert np.max(np.abs(back - vals)) < 1e-9
    out = torch.empty(n // 2, dtype=torch.complex128, device=dev)
    ctx.native.ckks_decode(pt, L, scale, out)
    assert np.max(np.abs(out.cpu().numpy() - vals)) < 1e-9
    sc = torch.empty(n, dtype=torch.int64, device=dev)
    ctx.native.ckks_encode_coeffs(dv, scale, sc)
    q0 = mods[0]
    want = [(x % q0) - q0 if x % q0 > q0 // 2 else x % q0 for x in X]
    assert [int(v) for v in sc.cpu().numpy()] == want


def test_encoder_bounds(dev):
    """The reference's bounds (src/ckks.cu:87-89, :122-126, :148-151): a
    scale whose bit count reaches the level's modulus, and coefficients whose
    bit count does, are refused; just below they are accepted."""
    import torch

    ph, ctx = make_ctx(12, [60, 50, 50, 50, 60], 1)
    n = ctx.N
    Q = 1
    for q in ctx.moduli[:4]:
        Q *= q
    tb = Q.bit_length()  # the level's total_coeff_modulus_bit_count
    v = torch.from_numpy(np.full(4, 0.5 + 0.25j)).to(dev)
    pt = empty((4, n), dev)
    ctx.native.ckks_encode(v, 2.0 ** (tb - 2), pt, 4)
    with pytest.raises(ValueError):
        ctx.native.ckks_encode(v, 2.0 ** (tb - 1), pt, 4)  # scale out of bounds
    with pytest.raises(ValueError):
        ctx.native.ckks_encode(torch.from_numpy(np.full(4, 1e30 + 0j)).to(dev), 2.0 ** (tb - 60), pt, 4)
    out = torch.empty(n // 2, dtype=torch.complex128, device=dev)
    with pytest.raises(ValueError):
        ctx.native.ckks_decode(pt, 4, 2.0 ** tb, out)


def test_encoder_errors(dev):
    ph, ctx = make_ctx(12, [60, 40, 60], 1)
    enc = ph.ckks_encoder(ctx)
    with pytest.raises(ValueError):
        enc.encode_double_vector(ctx, [], 2.0 ** 40)
    with pytest.raises(ValueError):
        enc.encode_double_vector(ctx, np.zeros(enc.slot_count() + 1), 2.0 ** 40)
    with pytest.raises(ValueError):
        enc.encode_double_vector(ctx, [1e30], 2.0 ** 40)  # coefficients of more bits than q0 q1


# ----------------------------------------------------------------- end to end
def test_reference_example_flow(dev):
    """python/examples/ckks.py of the reference, run against this module."""
    ph, ctx = make_ctx(14, [60, 40, 40, 60], 1, steps=[1, 2, 3, 4, 5, 6, 7])
    ph.set_seed(7)
    scale = 2.0 ** 40
    sk = ph.secret_key(ctx)
    pk = sk.gen_publickey(ctx)
    rlk = sk.gen_relinkey(ctx)
    glk = sk.create_galois_keys(ctx)
    enc = ph.ckks_encoder(ctx)
    slots = enc.slot_count()
    msg = [1.0, 2.0, 3.0, 4.0, 5.0, 6.0, 7.0, 8.0] + [0.0] * (slots - 8)
    pt = enc.encode_double_vector(ctx, msg, scale, chain_index=1)
    ct = pk.encrypt_asymmetric(ctx, pt)
    ct = ph.multiply_and_relin(ctx, ct, ct, rlk)
    ct = ph.rescale_to_next(ctx, ct)
    assert ct.chain_index() == 2
    ct2 = ph.hoisting(ctx, ct, glk, [1, 2, 3, 4, 5, 6, 7])
    ct = ph.add(ctx, ct, ct2)
    res = np.array(enc.decode_double_vector(ctx, sk.decrypt(ctx, ct)))
    sq = np.array(msg) ** 2
    want = sq + sum(np.roll(sq, -s) for s in range(1, 8))
    assert np.max(np.abs(res - want)) < 1e-4 * np.max(np.abs(want))
    assert np.max(np.abs(res - want)) < TOL * 64  # values up to 204, tolerance relative to 1e-6


@pytest.mark.parametrize("logN", [13, 16])
def test_mul_relin_rescale_decodes_within_1e6(dev, logN):
    """benchmark config 3 semantics at N = 2^16 (smaller chain for time): fresh
    ciphertexts of uniform reals in [-1, 1], HMult + relin + rescale, decode
    within 1e-6 absolute of the exact product."""
    ph, ctx = make_ctx(logN, [60] + [40] * 5 + [60] * 2, 2)
    ph.set_seed(logN)
    sk = ph.secret_key(ctx).generate_sparse(ctx, 192)
    rlk = sk.gen_relinkey(ctx)
    enc = ph.ckks_encoder(ctx)
    rng = np.random.default_rng(5)
    a = rng.uniform(-1, 1, enc.slot_count())
    b = rng.uniform(-1, 1, enc.slot_count())
    scale = 2.0 ** 40
    ca = sk.encrypt_symmetric(ctx, enc.encode_double_vector(ctx, a, scale))
    cb = sk.encrypt_symmetric(ctx, enc.encode_double_vector(ctx, b, scale))
    fresh = np.array(enc.decode_double_vector(ctx, sk.decrypt(ctx, ca)))
    assert np.max(np.abs(fresh - a)) < TOL
    c = ph.rescale_to_next(ctx, ph.multiply_and_relin(ctx, ca, cb, rlk))
    out = np.array(enc.decode_double_vector(ctx, sk.decrypt(ctx, c)))
    assert np.max(np.abs(out - a * b)) < TOL
    # the same through multiply (size 3) + relinearize
    c3 = ph.multiply(ctx, ca, cb)
    assert c3.size() == 3
    d3 = np.array(enc.decode_double_vector(ctx, sk.decrypt(ctx, c3)))  # size-3 decrypt uses s^2
    assert np.max(np.abs(d3 - a * b)) < TOL
    r = ph.rescale_to_next(ctx, ph.relinearize(ctx, c3, rlk))
    assert np.array_equal(to_host(r.data), to_host(c.data))
    # the fused single calls give the same ciphertext (residues, level and scale)
    for f in (ph.multiply_and_relin_rescale(ctx, ca, cb, rlk), ph.relinearize_rescale(ctx, c3, rlk)):
        assert np.array_equal(to_host(f.data), to_host(c.data))
        assert f.chain_index() == c.chain_index() and f.scale() == c.scale()


def test_rotations_and_conjugation(dev):
    """Rotations (direct and NAF) and conjugation decode within 1e-6.  The special
    modulus must dominate each key digit: hybrid key switching leaves an error
    ~ (Q_digit / P) (2N/pi) sigma sqrt(N) / scale in slot 0, because the ModUp
    digit is the uncentred residue in [0, Q_digit) (the oracle, i.e. the
    reference's algorithm, shows the same).  With one 60-bit special prime and a
    60-bit first digit that term alone is ~1e-6, so P = 2 x 60-bit here."""
    steps = [1, 2, 4, -1, 0]
    ph, ctx = make_ctx(13, [60, 40, 40, 40, 60, 60], 2, steps=steps)
    ph.set_seed(3)
    sk = ph.secret_key(ctx).generate_sparse(ctx, 192)  # the benchmark configs' sparse ternary secret
    glk = sk.create_galois_keys(ctx)
    enc = ph.ckks_encoder(ctx)
    rng = np.random.default_rng(8)
    v = rng.uniform(-1, 1, enc.slot_count()) + 1j * rng.uniform(-1, 1, enc.slot_count())
    ct = sk.encrypt_symmetric(ctx, enc.encode_complex_vector(ctx, v, 2.0 ** 40))
    for s in (1, 2, -1, 3, 5):  # 3 = 4 - 1 and 5 = 4 + 1 go through the NAF decomposition
        r = np.array(enc.decode_complex_vector(ctx, sk.decrypt(ctx, ph.rotate(ctx, ct, s, glk))))
        assert np.max(np.abs(r - np.roll(v, -s))) < TOL, s
    conj = np.array(enc.decode_complex_vector(ctx, sk.decrypt(ctx, ph.rotate(ctx, ct, 0, glk))))
    assert np.max(np.abs(conj - np.conj(v))) < TOL
    hs = ph.hoist_rotations(ctx, ct, glk, [1, 2, 4])
    for s, h in zip([1, 2, 4], hs):
        r = np.array(enc.decode_complex_vector(ctx, sk.decrypt(ctx, h)))
        assert np.max(np.abs(r - np.roll(v, -s))) < TOL
    with pytest.raises(RuntimeError):
        ph.hoist_rotations(ctx, ct, glk, [5])  # no key for step 5


def test_galois_keys_per_level(dev):
    """create_galois_keys_per_level / create_one_galois_key with a target chain
    index: keys with only the partitions that level needs rotate correctly
    there, are refused at a level that needs more, and the argument errors
    match the reference's exception classes."""
    ph, ctx = make_ctx(13, [60, 40, 40, 40, 40, 40, 60, 60], 2, steps=[1, 2])
    ph.set_seed(9)
    sk = ph.secret_key(ctx).generate_sparse(ctx, 192)
    enc = ph.ckks_encoder(ctx)
    assert ctx.dnum == 3
    g = sk.create_galois_keys_per_level(ctx, [0, 1], [3, 0])  # step 1 at chain index 3, step 2 full
    elt1, elt2 = ctx.galois_elts
    assert g.keys[elt1].shape[0] == 2 and g.keys[elt2].shape[0] == 3  # ceil(4 / 2) = 2 partitions
    rng = np.random.default_rng(10)
    v = rng.uniform(-1, 1, enc.slot_count())
    ct3 = sk.encrypt_symmetric(ctx, enc.encode_double_vector(ctx, v, 2.0 ** 40, chain_index=3))
    r = np.array(enc.decode_double_vector(ctx, sk.decrypt(ctx, ph.rotate(ctx, ct3, 1, g))))
    assert np.max(np.abs(r - np.roll(v, -1))) < TOL
    one = sk.create_one_galois_key(ctx, 0, 3)
    r = np.array(enc.decode_double_vector(ctx, sk.decrypt(ctx, ph.rotate_with_key(ctx, ct3, 1, one))))
    assert np.max(np.abs(r - np.roll(v, -1))) < TOL
    ct1 = sk.encrypt_symmetric(ctx, enc.encode_double_vector(ctx, v, 2.0 ** 40))
    with pytest.raises(ValueError):  # chain index 1 needs 3 partitions
        ph.rotate(ctx, ct1, 1, g)
    with pytest.raises(ValueError):
        sk.create_galois_keys_per_level(ctx, [0, 1], [3])
    with pytest.raises(IndexError):
        sk.create_one_galois_key(ctx, 2)
    with pytest.raises(ValueError):
        sk.create_one_galois_key(ctx, 0, ctx.size_Q + 1)
    # save writes one key per element in the context's order, whatever order
    # the indices were given in (PhantomGaloisKey::relin_keys_), so a load
    # gives every element its own key back
    import io

    perm = sk.create_galois_keys_per_level(ctx, [1, 0], [0, 3])
    buf = io.BytesIO()
    perm.save(buf)
    back = ph.galois_key().load(io.BytesIO(buf.getvalue()), ctx)
    for e in ctx.galois_elts:
        assert torch_equal(back.keys[e], perm.keys[e])
    r = np.array(enc.decode_double_vector(ctx, sk.decrypt(ctx, ph.rotate(ctx, ct3, 1, back))))
    assert np.max(np.abs(r - np.roll(v, -1))) < TOL
    r = np.array(enc.decode_double_vector(ctx, sk.decrypt(ctx, ph.rotate(ctx, ct1, 2, back))))
    assert np.max(np.abs(r - np.roll(v, -2))) < TOL
    # a set without a key for every element cannot be saved, as in the
    # reference (PhantomRelinKey::save of a key never generated)
    with pytest.raises(ValueError):
        sk.create_galois_keys_per_level(ctx, [1], [0]).save(io.BytesIO())


def torch_equal(a, b):
    import torch

    return a.shape == b.shape and bool(torch.equal(a, b))


def test_device_helpers(dev):
    import pyPhantom as ph

    n = ph.get_cuda_device_count()
    assert n >= 1
    ph.set_cuda_device(0)
    with pytest.raises(RuntimeError):
        ph.set_cuda_device(n)
    _, ctx = make_ctx(12, [60, 40, 60], 1)
    assert ctx.device == 0


@pytest.mark.parametrize("n,workgroups", [(2, 0), (2050, 0), (2050, 1), (2 * 35 * 65536, 0), (2 * 35 * 65536, 7)])
def test_stream_copy_exact(dev, n, workgroups):
    """pfa_stream_copy, the bench's copy ceiling: an exact copy of n words
    whatever the grid (a partial last group, a grid smaller than the data)."""
    import torch

    import pfa_native as P

    g = torch.Generator(device=dev)
    g.manual_seed(n + workgroups)
    src = torch.randint(-2 ** 62, 2 ** 62, (n,), dtype=torch.int64, device=dev, generator=g).view(torch.uint64)
    dst = torch.zeros_like(src)
    P.stream_copy(dst, src, workgroups)
    torch.cuda.synchronize()
    assert torch.equal(dst.view(torch.int64), src.view(torch.int64))


def test_stream_copy_errors(dev):
    import torch

    import pfa_native as P

    a = torch.zeros(8, dtype=torch.int64, device=dev).view(torch.uint64)
    b = torch.zeros(8, dtype=torch.int64, device=dev).view(torch.uint64)
    with pytest.raises(ValueError):
        P.stream_copy(a, b[:7])  # sizes differ
    with pytest.raises(ValueError):
        P.stream_copy(a[:7], b[:7])  # odd length
    with pytest.raises(ValueError):
        P.stream_copy(a[1:7], b[1:7])  # 8-byte aligned only


def test_cuda_stream_runs_calls_on_its_stream(dev):
    """cuda_stream (binding.cu:69-70): calls made inside `with cuda_stream()` run
    on that stream and give the residues the default stream gives; results
    made on it are read correctly from the default stream afterwards."""
    import torch

    ph, ctx = make_ctx(13, [60, 40, 40, 60], 1)
    ph.set_seed(3)
    sk = ph.secret_key(ctx)
    rlk = sk.gen_relinkey(ctx)
    enc = ph.ckks_encoder(ctx)
    rng = np.random.default_rng(8)
    a = rng.uniform(-1, 1, enc.slot_count())
    ca = sk.encrypt_symmetric(ctx, enc.encode_double_vector(ctx, a, 2.0 ** 40))
    want = to_host(ph.multiply_and_relin_rescale(ctx, ca, ca, rlk).data)
    s = ph.cuda_stream()
    assert s.stream != torch.cuda.current_stream()
    with s:
        assert torch.cuda.current_stream() == s.stream
        got = ph.multiply_and_relin_rescale(ctx, ca, ca, rlk)
    assert torch.cuda.current_stream() != s.stream
    assert np.array_equal(to_host(got.data), want)
    out = np.array(enc.decode_double_vector(ctx, sk.decrypt(ctx, got)))
    assert np.max(np.abs(out - a * a)) < TOL


def test_api_errors(dev):
    ph, ctx = make_ctx(12, [60, 40, 40, 60], 1)
    sk = ph.secret_key(ctx)
    enc = ph.ckks_encoder(ctx)
    c1 = sk.encrypt_symmetric(ctx, enc.encode_double_vector(ctx, [1.0], 2.0 ** 30))
    c2 = sk.encrypt_symmetric(ctx, enc.encode_double_vector(ctx, [1.0], 2.0 ** 30, chain_index=2))
    with pytest.raises(ValueError):
        ph.add(ctx, c1, c2)
    with pytest.raises(ValueError):
        ph.rescale_to_next(ctx, ph.rescale_to_next(ctx, ph.rescale_to_next(ctx, c1)))
    with pytest.raises(ValueError):
        ph.params(ph.scheme_type.bfv)


def test_serialization_reference_layout(dev):
    """save/load in the reference's binary layout (include/ciphertext.h:173-214,
    include/plaintext.h:73-101, include/secretkey.h:99-111, :192-228, :290-318,
    :537-575): the headers carry the reference's fields in its order, the
    objects round-trip exactly, and loaded keys work."""
    import io
    import struct

    import torch

    ph, ctx = make_ctx(12, [60, 40, 40, 60], 1, steps=[1, -1])
    ph.set_seed(21)
    sk = ph.secret_key(ctx).generate_sparse(ctx, 64)
    pk = sk.gen_publickey(ctx)
    rlk = sk.gen_relinkey(ctx)
    glk = sk.create_galois_keys(ctx)
    enc = ph.ckks_encoder(ctx)
    rng = np.random.default_rng(22)
    v = rng.uniform(-1, 1, enc.slot_count())
    pt = enc.encode_double_vector(ctx, v, 2.0 ** 40)
    ct = sk.encrypt_symmetric(ctx, pt)
    N, L, QP = ctx.N, ctx.size_Ql(1), len(ctx.moduli)

    # ciphertext: 7 x 8-byte fields + 2 bools (58 bytes), then [2][L][N] uint64
    buf = io.BytesIO()
    ct.save(buf)
    raw = buf.getvalue()
    assert len(raw) == 58 + 2 * L * N * 8
    assert struct.unpack("<QQQQdQQ??", raw[:58]) == (1, 2, N, L, 2.0 ** 40, 1, 1, True, False)
    assert raw[58:66] == to_host(ct.data)[0, 0, 0].tobytes()
    ct2 = ph.ciphertext().load(io.BytesIO(raw), ctx)
    assert torch.equal(ct2.data, ct.data) and ct2.chain_index() == 1 and ct2.scale() == ct.scale()

    # plaintext: chain, N, L, scale, then [L][N]
    buf = io.BytesIO()
    pt.save(buf)
    raw = buf.getvalue()
    assert len(raw) == 32 + L * N * 8 and struct.unpack("<QQQd", raw[:32]) == (1, N, L, 2.0 ** 40)
    assert torch.equal(ph.plaintext().load(io.BytesIO(raw), ctx).data, pt.data)

    # secret key: power 1, N, |QP|, then s over every prime
    buf = io.BytesIO()
    sk.save(buf)
    raw = buf.getvalue()
    assert struct.unpack("<QQQ", raw[:24]) == (1, N, QP) and len(raw) == 24 + QP * N * 8
    sk2 = ph.secret_key().load(io.BytesIO(raw), ctx)
    got = np.array(enc.decode_double_vector(ctx, sk2.decrypt(ctx, ct2)))
    assert np.max(np.abs(got - v)) < 1e-6

    # public key: one key-level ciphertext record [2][QP][N]
    buf = io.BytesIO()
    pk.save(buf)
    raw = buf.getvalue()
    assert struct.unpack("<QQQQdQQ??", raw[:58])[:4] == (0, 2, N, QP)
    pk2 = ph.public_key().load(io.BytesIO(raw), ctx)
    got = np.array(enc.decode_double_vector(ctx, sk.decrypt(ctx, pk2.encrypt_asymmetric(ctx, pt))))
    assert np.max(np.abs(got - v)) < 1e-6

    # relin key: dnum, then dnum key-level ciphertexts; galois key: count, then relin keys
    buf = io.BytesIO()
    rlk.save(buf)
    raw = buf.getvalue()
    dnum = int(rlk.data.shape[0])
    assert struct.unpack("<Q", raw[:8]) == (dnum,) and len(raw) == 8 + dnum * (58 + 2 * QP * N * 8)
    rlk2 = ph.relin_key().load(io.BytesIO(raw), ctx)
    assert torch.equal(rlk2.data, rlk.data)
    y1 = ph.multiply_and_relin(ctx, ct, ct, rlk)
    y2 = ph.multiply_and_relin(ctx, ct2, ct2, rlk2)
    assert torch.equal(y1.data, y2.data)
    buf = io.BytesIO()
    glk.save(buf)
    raw = buf.getvalue()
    assert struct.unpack("<Q", raw[:8]) == (len(ctx.galois_elts),)
    glk2 = ph.galois_key().load(io.BytesIO(raw), ctx)
    assert list(glk2.keys) == list(glk.keys)
    assert torch.equal(ph.rotate(ctx, ct, 1, glk2).data, ph.rotate(ctx, ct, 1, glk).data)

    # a truncated stream or a corrupt header is an error, not a short object
    buf = io.BytesIO()
    ct.save(buf)
    raw = buf.getvalue()
    with pytest.raises(ValueError):
        ph.ciphertext().load(io.BytesIO(raw[:-8]), ctx)
    with pytest.raises(ValueError):
        ph.ciphertext().load(io.BytesIO(struct.pack("<QQQQdQQ??", 1, 2, 0, L, 1.0, 1, 1, True, False)), ctx)


def test_single_chain_plaintext_api(dev):
    """encode_single_chain_plaintext / expand_single_chain_to_full
    (src/single_chain_plaintext.cu:93-192) and the bytes round trip of the
    Python binding (python/src/binding.cu:405-519): the expansion at a level
    equals encode at that level, residue for residue."""
    import torch

    ph, ctx = make_ctx(13, [60, 40, 40, 60], 1)
    enc = ph.ckks_encoder(ctx)
    rng = np.random.default_rng(23)
    v = rng.uniform(-1, 1, enc.slot_count()) + 1j * rng.uniform(-1, 1, enc.slot_count())
    scale = 2.0 ** 40
    scp = ph.encode_single_chain_plaintext(ctx, enc, v, scale)
    assert scp.N == ctx.N and scp.nbytes == 8 * ctx.N and scp.scale == scale == scp.get_scale()
    for chain in (1, 2):
        full = ph.expand_single_chain_to_full(ctx, scp, chain)
        ref = enc.encode_complex_vector(ctx, v, scale, chain)
        assert full.chain_index() == chain and full.scale() == scale
        assert torch.equal(full.data, ref.data)
    scp2 = ph.scp_from_bytes(scp.coeffs_bytes(), scale, ctx.N, ctx)
    assert torch.equal(ph.expand_single_chain_to_full(ctx, scp2, 1).data,
                       ph.expand_single_chain_to_full(ctx, scp, 1).data)
    with pytest.raises(RuntimeError):
        ph.scp_from_bytes(b"\0" * 8, scale, ctx.N, ctx)


def test_library_loaded_before_torch(dev):
    """A fresh process that uses pyPhantom without importing torch itself: the
    loader imports torch before the library, so both share torch's HIP runtime
    and the device is visible to both."""
    import os
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    code = (
        "import sys; sys.path[:0] = [%r, %r]\n"
        "import numpy as np, pyPhantom as ph\n"
        "p = ph.params(ph.scheme_type.ckks); N = 1 << 12\n"
        "p.set_poly_modulus_degree(N); p.set_coeff_modulus(ph.create_coeff_modulus(N, [60, 40, 60]))\n"
        "p.set_special_modulus_size(1); ctx = ph.context(p); enc = ph.ckks_encoder(ctx)\n"
        "z = np.linspace(-1, 1, N // 2)\n"
        "got = enc.decode_double_vector(ctx, enc.encode_double_vector(ctx, z, 2.0 ** 40))\n"
        "print('max err', float(np.max(np.abs(np.array(got) - z))))\n"
    ) % (root, os.path.join(root, "phantom-fhe_amd"))
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr[-2000:]
    assert float(r.stdout.split()[-1]) < 1e-6


@pytest.mark.parametrize("logN,batch,L,start", [(16, 2, 35, 0), (13, 1, 3, 1), (12, 3, 4, 2)])
def test_pyphantom_ntt_entry_points(dev, logN, batch, L, start):
    """pyPhantom.ntt_forward / ntt_inverse (the C++ nwt_2d_radix8_forward_inplace
    [_batched] / nwt_2d_radix8_backward_inplace signatures, include/ntt.cuh:173,
    :184, :216) against the oracle, including a start offset into the table and
    the config-2 batch; then the argument errors."""
    N = 1 << logN
    bits = [50] * 35 + [60] if logN == 16 else [60, 50, 55, 60, 49, 60]
    ph, ctx = make_ctx(logN, bits, 1)
    orc = O.Oracle(N, ctx.moduli, 1)
    rng = np.random.default_rng(logN + L)
    x = uniform_limbs(rng, (batch, L, N), ctx.moduli[start:start + L])
    d = to_dev(x, dev)
    ph.ntt_forward(ctx, d, L, start, batch)
    ph.synchronize(ctx)
    got, want = to_host(d), orc.ntt_fwd(x, start=start, threads=8)
    assert np.array_equal(got, want), first_mismatch(got, want)
    ph.ntt_inverse(ctx, d, L, start, batch)
    back = to_host(d)
    assert np.array_equal(back, x), first_mismatch(back, x)
    with pytest.raises(ValueError):  # size does not match batch x L x N
        ph.ntt_forward(ctx, d, L + 1, start, batch)
    with pytest.raises(ValueError):  # limbs beyond the context's primes
        ph.ntt_forward(ctx, empty((batch, len(ctx.moduli), N), dev), len(ctx.moduli), 1, batch)
    with pytest.raises(ValueError):  # not a uint64 tensor
        ph.ntt_forward(ctx, d.view(torch_int64()), L, start, batch)


def torch_int64():
    import torch

    return torch.int64


def test_ct_multiply_plain_matches_per_poly(dev):
    """pfa_ct_multiply_plain (multiply_plain_ntt, src/evaluate.cu:1224-1250) over
    4 polys in one launch equals poly_mul per poly, in place too; 50- and
    60-bit primes (both arithmetic policies)."""
    import pfa_native as P

    N = 1 << 12
    mods = O.create_coeff_modulus(N, [60, 50, 55, 60])
    ctx = P.NativeContext(N, mods, 1)
    rng = np.random.default_rng(4)
    L = 3
    ct = uniform_limbs(rng, (4, L, N), mods[:L])
    pt = uniform_limbs(rng, (L, N), mods[:L])
    dct, dpt = to_dev(ct, dev), to_dev(pt, dev)
    out = empty((4, L, N), dev)
    ctx.ct_multiply_plain(dct, dpt, out, L)
    want = np.stack([np.stack([(ct[k, l].astype(object) * pt[l].astype(object)) % mods[l] for l in range(L)])
                     for k in range(4)]).astype(np.uint64)
    assert np.array_equal(to_host(out), want)
    ctx.ct_multiply_plain(dct, dpt, dct, L)
    assert np.array_equal(to_host(dct), want)
