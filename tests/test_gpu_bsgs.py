"""GPU tests of the BSGS encrypted matrix-vector product (include/bsgs.h,
src/bsgs.cu) and its C-ABI pieces.

* pfa_bsgs_mac (every giant's accumulation in one launch) is bit-exact against
  the oracle's elementwise products summed mod q, on both arithmetic policies.
* pfa_ckks_encode_coeffs + pfa_expand_signed + the forward NTT reproduce
  pfa_ckks_encode residue for residue (the single-chain plaintext route the
  reference takes, src/single_chain_plaintext.cu:93-150, src/bsgs.cu:245-271).
* The whole product (babies by chained power-of-two rotations, giants by
  Horner rotations, one rescale) is bit-exact against the same algorithm run on
  the oracle from the same key material, plaintext coefficients and input
  ciphertext, and its decryption matches W x within a tolerance.
The reference ships no BSGS vectors (its bsgs test checks decode error only,
python/llm_project/blocks/bsgs_test.py:77), so the residues are pinned by the
oracle composition and the values by numpy.
"""
import numpy as np
import pytest

import py_oracle as O
from gpu_util import empty, first_mismatch, to_dev, to_host, uniform_limbs

pytestmark = pytest.mark.gpu


def make_ctx(logN, bits, special, steps=()):
    import pyPhantom as ph

    N = 1 << logN
    p = ph.params(ph.scheme_type.ckks)
    p.set_poly_modulus_degree(N)
    p.set_coeff_modulus(ph.create_coeff_modulus(N, bits))
    p.set_special_modulus_size(special)
    p.set_galois_elts(ph.get_elts_from_steps(list(steps), N))
    return ph, ph.context(p)


def add_mod(a, b, mods):
    out = a + b  # residues below 2^61: no uint64 overflow
    for l, q in enumerate(mods):
        out[..., l, :] %= np.uint64(q)
    return out


@pytest.mark.parametrize("M,G,chain", [(5, 3, 1), (8, 1, 2), (1, 4, 1), (9, 2, 1), (3, 19, 1), (70, 2, 1)])
def test_bsgs_mac_matches_oracle(dev, M, G, chain):
    import pfa_native as P

    N = 1 << 12
    mods = O.create_coeff_modulus(N, [60, 50, 45, 60, 50, 60])
    ctx = P.NativeContext(N, mods, 1)
    orc = O.Oracle(N, mods, 1)
    Ql = orc.size_Ql(chain)
    qs = mods[:Ql]
    rng = np.random.default_rng(M * 10 + G + chain)
    pts = [uniform_limbs(rng, (Ql, N), qs) for _ in range(M * G)]
    babies = [uniform_limbs(rng, (2, Ql, N), qs) for _ in range(M)]
    dpts = [to_dev(p, dev) for p in pts]
    dbab = [to_dev(b, dev) for b in babies]
    outs = [empty((2, Ql, N), dev) for _ in range(G)]
    ctx.bsgs_mac(chain, dpts, dbab, outs)
    for g in range(G):
        want = np.zeros((2, Ql, N), dtype=np.uint64)
        for b in range(M):
            for k in range(2):
                want[k] = add_mod(want[k], orc.mul_poly(pts[g * M + b], babies[b][k]), qs)
        got = to_host(outs[g])
        assert np.array_equal(got, want), (g, first_mismatch(got, want))


@pytest.mark.parametrize("M,G,chunk", [(4, 19, 7), (64, 2, 128), (1, 9, 9)])
def test_bsgs_tiled_mac_equals_pointer_mac(dev, M, G, chunk):
    """The tiled plaintext layout, filled in chunks, gives the same sums as the
    pointer-list accumulation (and so as the oracle)."""
    import pfa_native as P
    import torch

    N = 1 << 12
    mods = O.create_coeff_modulus(N, [60, 50, 45, 60, 50, 60])
    ctx = P.NativeContext(N, mods, 1)
    chain = 1
    Ql = len(mods) - 1
    rng = np.random.default_rng(M + G)
    D = M * G
    pts = to_dev(np.stack([uniform_limbs(rng, (Ql, N), mods[:Ql]) for _ in range(D)]), dev)
    babies = [to_dev(uniform_limbs(rng, (2, Ql, N), mods[:Ql]), dev) for _ in range(M)]
    tiled = empty((D * Ql * N,), dev)
    for d0 in range(0, D, chunk):
        n = min(chunk, D - d0)
        ctx.bsgs_tile_plaintexts(chain, pts[d0:d0 + n], n, tiled, d0, D)
    # the layout itself: limb j, span t of plaintext d at ((j T + t) D + d) 512
    T = N // 512
    view = tiled.view(Ql, T, D, 512)
    d, j, t = D - 1, Ql - 1, T - 1
    assert torch.equal(view[j, t, d], pts[d, j, t * 512:(t + 1) * 512])
    want = [empty((2, Ql, N), dev) for _ in range(G)]
    got = [empty((2, Ql, N), dev) for _ in range(G)]
    ctx.bsgs_mac(chain, [pts[i] for i in range(D)], babies, want)
    ctx.bsgs_mac_tiled(chain, tiled, babies, got)
    for g in range(G):
        assert torch.equal(got[g], want[g]), g


@pytest.mark.parametrize("M,G", [(8, 5), (64, 2)])
def test_bsgs_tiled_packed_limbs(dev, M, G):
    """Limbs whose prime is below 2^40 are stored in 5 bytes per residue in the
    tiled set; the accumulation over such a set equals the pointer-list one, and
    the set's size is 5 / 8 of the unpacked size on those limbs."""
    import pfa_native as P
    import torch

    N = 1 << 12
    mods = O.create_coeff_modulus(N, [60, 40, 38, 40, 50, 40, 60])
    ctx = P.NativeContext(N, mods, 1)
    chain = 1
    Ql = len(mods) - 1
    D = M * G
    packed = sum(1 for q in mods[:Ql] if q < (1 << 40))
    assert packed == 4
    assert ctx.bsgs_tiled_size(chain, D) == D * N * (5 * packed + 8 * (Ql - packed))
    rng = np.random.default_rng(M * G + 1)
    pts = uniform_limbs(rng, (D, Ql, N), mods[:Ql])
    pts[0, 1, :4] = [0, mods[1] - 1, (1 << 32) - 1, 1 << 32]  # the packing's edges
    dpts = to_dev(pts, dev)
    babies = [to_dev(uniform_limbs(rng, (2, Ql, N), mods[:Ql]), dev) for _ in range(M)]
    tiled = empty(((ctx.bsgs_tiled_size(chain, D) + 7) // 8,), dev)
    ctx.bsgs_tile_plaintexts(chain, dpts, D, tiled, 0, D)
    want = [empty((2, Ql, N), dev) for _ in range(G)]
    got = [empty((2, Ql, N), dev) for _ in range(G)]
    ctx.bsgs_mac(chain, [dpts[i] for i in range(D)], babies, want)
    ctx.bsgs_mac_tiled(chain, tiled, babies, got)
    for g in range(G):
        assert torch.equal(got[g], want[g]), g


def test_bsgs_tiled_packed_mac_config4_full_size(dev):
    """The accumulation config 4 runs (tiled set, its 19 limbs of 40 bits
    packed to 5 bytes, the 60-bit limb in the integer policy) at N = 2^16 on
    config 4's chain, against the oracle's products summed mod q: 16 babies
    and 3 giants of the real 64 x 64."""
    import pfa_native as P

    N = 1 << 16
    mods = O.create_coeff_modulus(N, [60] + [40] * 19 + [60] * 4)
    ctx = P.NativeContext(N, mods, 4)
    orc = O.Oracle(N, mods, 4)
    chain, M, G = 1, 16, 3
    Ql = orc.size_Ql(chain)
    qs = mods[:Ql]
    D = M * G
    rng = np.random.default_rng(404)
    pts = uniform_limbs(rng, (D, Ql, N), qs)
    babies = [uniform_limbs(rng, (2, Ql, N), qs) for _ in range(M)]
    tiled = empty(((ctx.bsgs_tiled_size(chain, D) + 7) // 8,), dev)
    ctx.bsgs_tile_plaintexts(chain, to_dev(pts, dev), D, tiled, 0, D)
    got = [empty((2, Ql, N), dev) for _ in range(G)]
    ctx.bsgs_mac_tiled(chain, tiled, [to_dev(b, dev) for b in babies], got)
    for g in range(G):
        want = np.zeros((2, Ql, N), dtype=np.uint64)
        for b in range(M):
            for k in range(2):
                want[k] = add_mod(want[k], orc.mul_poly(pts[g * M + b], babies[b][k]), qs)
        h = to_host(got[g])
        assert np.array_equal(h, want), (g, first_mismatch(h, want))


def test_bsgs_mac_rejects_bad_arguments(dev):
    import pfa_native as P

    N = 1 << 12
    mods = O.create_coeff_modulus(N, [60, 50, 60])
    ctx = P.NativeContext(N, mods, 1)
    x = empty((2, 2, N), dev)
    with pytest.raises(ValueError):
        ctx.bsgs_mac(1, [x[0]], [x], [])  # no giants
    with pytest.raises(ValueError):
        ctx.bsgs_mac(5, [x[0]], [x], [x])  # chain index out of range
    with pytest.raises(ValueError):
        ctx.bsgs_tile_plaintexts(1, x[0], 2, x, 1, 2)  # positions past the set
    with pytest.raises(ValueError):
        ctx.bsgs_giants(2, x, 1, 1, None, x)  # rescale at the last level
    with pytest.raises(ValueError):
        ctx.bsgs_giants(1, x, 2, 1, None, x)  # a rotation without a key
    with pytest.raises(ValueError):
        ctx.bsgs_babies(1, x, 2, [empty((0, 2, 3, N), dev)], empty((2, 2, 2, N), dev))  # key without digits
    with pytest.raises(ValueError):
        ctx.bsgs_babies(3, x, 2, [x], x)  # chain index out of range
    with pytest.raises(ValueError):
        ctx.bsgs_apply_giants(1, x, [x], 2, None, x)  # a rotation without a key
    with pytest.raises(ValueError):
        ctx.bsgs_apply_giants(2, x, [x], 1, None, x)  # rescale at the last level


def test_single_chain_encode_expand_equals_encode(dev):
    import torch

    ph, ctx = make_ctx(13, [60, 40, 40, 60], 1)
    enc = ph.ckks_encoder(ctx)
    rng = np.random.default_rng(3)
    v = rng.uniform(-1, 1, enc.slot_count()) + 1j * rng.uniform(-1, 1, enc.slot_count())
    scale = 2.0 ** 40
    L = ctx.size_Ql(1)
    ref = enc.encode_complex_vector(ctx, v, scale)
    coeffs = torch.empty(ctx.N, dtype=torch.int64, device=ctx.dev)
    ctx.native.ckks_encode_coeffs(torch.from_numpy(v).to(ctx.dev), scale, coeffs)
    c = coeffs.cpu().numpy()
    assert np.max(np.abs(c)) < 2 ** 62
    out = ctx._empty(1, L, ctx.N)
    ctx.native.expand_signed(coeffs.view(1, -1), 1, out, L)
    want = np.stack([np.mod(c, q).astype(np.uint64) for q in ctx.moduli[:L]])
    assert np.array_equal(to_host(out[0]), want)
    ctx.native.ntt_forward(out, 1, L, 0)
    assert np.array_equal(to_host(out[0]), to_host(ref.data))


def _oracle_bsgs(orc, mods, chain, x, glk_host, P, M, G, N):
    """The reference's algorithm (src/bsgs.cu:195-333) on the oracle."""
    from pyPhantom import get_elt_from_step

    def rot(ct, ch, step):
        e = get_elt_from_step(step, N)
        return orc.apply_galois(ch, ct, e, glk_host[e], threads=8)

    Ql = orc.size_Ql(chain)
    qs = mods[:Ql]
    babies = [x]
    for b in range(1, M):
        bit = 1 << (b.bit_length() - 1)
        babies.append(rot(babies[b - bit], chain, bit))
    partial = []
    for g in range(G):
        acc = np.zeros((2, Ql, N), dtype=np.uint64)
        for b in range(M):
            for k in range(2):
                acc[k] = add_mod(acc[k], orc.mul_poly(P[g * M + b], babies[b][k]), qs)
        partial.append(acc)
    acc = partial[G - 1]
    for g in range(G - 2, -1, -1):
        acc = add_mod(rot(acc, chain, M), partial[g], qs)
    return orc.rescale(chain, acc, threads=8)


@pytest.mark.parametrize("M,G,rows,cols", [(8, 8, 48, 40), (1, 8, 8, 6), (4, 1, 3, 4)])
def test_bsgs_matmul_bit_exact_and_decodes(dev, M, G, rows, cols):
    """d_pad = M G at N = 2^12 (2048 slots), a rows x cols matrix (zero padding
    in both directions), x in replicated-block layout.  The GPU result equals
    the oracle's run of the same algorithm and decrypts to W x; the babies and
    the giant stage equal the evaluator's own rotate / add composition."""
    import torch

    d_pad = M * G
    ph, ctx = make_ctx(12, [60, 40, 40, 40, 60, 60], 2, steps=[1, 2, 4, 8])
    assert set(ph.bsgs_required_steps(M)) <= {1, 2, 4, 8}
    ph.set_seed(11)
    sk = ph.secret_key(ctx).generate_sparse(ctx, 64)
    glk = sk.create_galois_keys(ctx)
    enc = ph.ckks_encoder(ctx)
    slots = enc.slot_count()
    rng = np.random.default_rng(12 + M)
    W = rng.uniform(-1 / 8, 1 / 8, (rows, cols))
    xv = np.zeros(d_pad)
    xv[:cols] = rng.uniform(-1, 1, cols)
    scale = 2.0 ** 40
    diags = ph.pre_encode_bsgs_diagonals(ctx, enc, W.ravel(), rows, cols, d_pad, M, scale)
    assert (diags.d_pad, diags.baby_steps, diags.giant_steps) == (d_pad, M, G)
    x = sk.encrypt_symmetric(ctx, enc.encode_double_vector(ctx, np.tile(xv, slots // d_pad), scale))
    y = ph.bsgs_matmul_preencoded(ctx, glk, x, diags)
    assert y.chain_index() == 2 and y.scale() == x.scale()

    # decrypted values: y[i] = (W x)[i] for i < rows, 0 on the pad, every period
    want = np.zeros(d_pad)
    want[:rows] = W @ xv[:cols]
    got = np.array(enc.decode_double_vector(ctx, sk.decrypt(ctx, y)))
    err = np.max(np.abs(got - np.tile(want, slots // d_pad)))
    assert err < 1e-5, err

    # residues against the oracle running the reference's algorithm
    orc = O.Oracle(ctx.N, ctx.moduli, ctx.size_P)
    L = ctx.size_Ql(1)
    c = diags.coeffs.cpu().numpy()
    P = [orc.ntt_fwd(np.stack([np.mod(c[d], q).astype(np.uint64) for q in ctx.moduli[:L]])[None])[0]
         for d in range(d_pad)]
    keys = {e: to_host(k) for e, k in glk.keys.items()}
    want_res = _oracle_bsgs(orc, ctx.moduli, 1, to_host(x.data), keys, P, M, G, ctx.N)
    got_res = to_host(y.data)
    assert np.array_equal(got_res, want_res), first_mismatch(got_res, want_res)

    # babies + giants split (compute_bsgs_babies / bsgs_apply_giants_with_babies) give the same
    babies = ph.compute_bsgs_babies(ctx, glk, x, M)
    y2 = ph.bsgs_apply_giants_with_babies(ctx, glk, babies, diags)
    assert torch.equal(y2.data, y.data)

    # the native baby chain equals rotate() one step at a time
    for b in range(1, M):
        bit = 1 << (b.bit_length() - 1)
        assert torch.equal(babies[b].data, ph.rotate(ctx, babies[b - bit], bit, glk).data), b

    # the native giant stage equals rotate / add / rescale_to_next on the same partials
    partials = ctx._empty(G, 2, L, ctx.N)
    ctx.native.bsgs_mac_tiled(1, diags.expanded(ctx, 1), [b.data for b in babies], [partials[g] for g in range(G)])
    acc = x._like(partials[G - 1])
    for g in range(G - 2, -1, -1):
        acc = ph.add(ctx, ph.rotate(ctx, acc, M, glk), x._like(partials[g]))
    assert torch.equal(ph.rescale_to_next(ctx, acc).data, y.data)
    # and so does the Horner-only entry point on the same partials
    out = ctx._empty(2, L - 1, ctx.N)
    key = glk.get(ph.get_elt_from_step(M, ctx.N)) if G > 1 else None
    ctx.native.bsgs_giants(1, partials, G, M, key, out)
    assert torch.equal(out, y.data)


@pytest.mark.parametrize("M", [6, 70])
def test_bsgs_babies_any_count(dev, M):
    """compute_bsgs_babies for baby counts that are not powers of two and above
    the 64 babies passed by value (the reference takes any count,
    src/bsgs.cu:194-214): the batched native chain equals rotate() one step
    at a time."""
    import torch

    steps = [1 << k for k in range((M - 1).bit_length())]
    ph, ctx = make_ctx(12, [60, 40, 40, 60], 1, steps=steps)
    ph.set_seed(5)
    sk = ph.secret_key(ctx).generate_sparse(ctx, 64)
    glk = sk.create_galois_keys(ctx)
    enc = ph.ckks_encoder(ctx)
    rng = np.random.default_rng(M)
    x = sk.encrypt_symmetric(ctx, enc.encode_double_vector(ctx, rng.uniform(-1, 1, enc.slot_count()), 2.0 ** 40))
    babies = ph.compute_bsgs_babies(ctx, glk, x, M)
    assert len(babies) == M and babies[0] is x
    for b in range(1, M):
        bit = 1 << (b.bit_length() - 1)
        assert torch.equal(babies[b].data, ph.rotate(ctx, babies[b - bit], bit, glk).data), b


@pytest.mark.parametrize("mode", ["Rows", "ColsConj"])
def test_bsgs_complex_fold_decodes(dev, mode):
    """pre_encode_bsgs_diagonals_complex (src/bsgs.cu:415-514) + the complex
    product: Rows packs (W x)[i] and (W x)[i + ceil(R/2)] into one slot's real
    and imaginary parts; ColsConj takes x packed as x[j] + i x[j + ceil(C/2)]
    and returns W x in the real parts."""
    M, G = 4, 4
    d_pad = M * G
    R, C = (24, 12) if mode == "Rows" else (10, 20)
    ph, ctx = make_ctx(12, [60, 40, 40, 40, 60, 60], 2, steps=[1, 2, 4])
    ph.set_seed(13)
    sk = ph.secret_key(ctx).generate_sparse(ctx, 64)
    glk = sk.create_galois_keys(ctx)
    enc = ph.ckks_encoder(ctx)
    slots = enc.slot_count()
    rng = np.random.default_rng(14)
    W = rng.uniform(-1 / 8, 1 / 8, (R, C))
    x = rng.uniform(-1, 1, C)
    scale = 2.0 ** 40
    fold = getattr(ph.ComplexFoldMode, mode)
    diags = ph.pre_encode_bsgs_diagonals_complex(ctx, enc, W.ravel(), R, C, d_pad, M, scale, fold)
    xv = np.zeros(d_pad, dtype=np.complex128)
    if mode == "Rows":
        xv[:C] = x
    else:
        h = (C + 1) // 2
        xv[:h] = x[:h]
        xv[:C - h] += 1j * x[h:]
    ct = sk.encrypt_symmetric(ctx, enc.encode_complex_vector(ctx, np.tile(xv, slots // d_pad), scale))
    y = ph.bsgs_matmul_preencoded_complex(ctx, glk, ct, diags)
    got = np.array(enc.decode_complex_vector(ctx, sk.decrypt(ctx, y)))[:d_pad]
    want = W @ x
    if mode == "Rows":
        h = (R + 1) // 2
        assert np.max(np.abs(got[:h].real - want[:h])) < 1e-5
        assert np.max(np.abs(got[:R - h].imag - want[h:])) < 1e-5
    else:
        assert np.max(np.abs(got[:R].real - want)) < 1e-5
    # the split API gives the same residues
    babies = ph.compute_bsgs_babies(ctx, glk, ct, M)
    y2 = ph.bsgs_apply_giants_with_babies_complex(ctx, glk, babies, diags)
    import torch
    assert torch.equal(y2.data, y.data)


def test_bsgs_argument_checks(dev):
    ph, ctx = make_ctx(12, [60, 40, 60], 1)
    enc = ph.ckks_encoder(ctx)
    W = np.zeros((4, 4))
    with pytest.raises(ValueError):
        ph.pre_encode_bsgs_diagonals(ctx, enc, W.ravel(), 4, 4, 6, 2, 2.0 ** 30)  # d_pad not a power of 2
    with pytest.raises(ValueError):
        ph.pre_encode_bsgs_diagonals(ctx, enc, W.ravel(), 4, 4, 2, 1, 2.0 ** 30)  # d_pad < dims
    with pytest.raises(ValueError):
        ph.pre_encode_bsgs_diagonals(ctx, enc, W.ravel(), 4, 4, 8, 3, 2.0 ** 30)  # baby steps must divide
    with pytest.raises(ValueError):
        ph.pre_encode_bsgs_diagonals(ctx, enc, W.ravel()[:15], 4, 4, 8, 2, 2.0 ** 30)  # size mismatch
    with pytest.raises(ValueError):  # folded 4 x 2 needs d_pad >= 4
        ph.pre_encode_bsgs_diagonals_complex(ctx, enc, W.ravel(), 4, 4, 2, 1, 2.0 ** 30, ph.ComplexFoldMode.ColsConj)
