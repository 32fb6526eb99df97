"""Pins the CPU oracle (oracle/ckks_oracle.c) before it is trusted as the checker.

The reference ships no golden vectors for this path (its NTT test only
round-trips constant inputs, test/ntt_test.cu:48-50, :103-106), so every
oracle function is pinned here against what the mathematics fixes: closed
forms evaluated with Python big integers, brute force on small inputs,
CRT identities and the scheme's decryption invariant.  Each check is chosen
so a plausible slip (wrong root, wrong bit-reversal, missing N^-1 fold,
wrong partition, corrected vs uncorrected base conversion, rounding vs floor
rescale, wrong Galois index) fails it.
"""
import random

import numpy as np
import pytest

import py_oracle as O

N_SMALL = 64


# ----------------------------------------------------------------- helpers
def mr_prime(n: int) -> bool:
    """Independent primality test (trial division + Miller-Rabin, bases != oracle's loop)."""
    if n < 2:
        return False
    for p in (2, 3, 5, 7, 11, 13, 17, 19, 23, 29, 31, 37, 41, 43, 47):
        if n % p == 0:
            return n == p
    d, r = n - 1, 0
    while d % 2 == 0:
        d //= 2
        r += 1
    for a in (2, 325, 9375, 28178, 450775, 9780504, 1795265022):
        if a % n == 0:
            continue
        x = pow(a, d, n)
        if x in (1, n - 1):
            continue
        for _ in range(r - 1):
            x = x * x % n
            if x == n - 1:
                break
        else:
            return False
    return True


def brv(x: int, bits: int) -> int:
    return int(bin(x)[2:].zfill(bits)[::-1], 2) if bits else 0


def negacyclic_mul(a, b, q):
    n = len(a)
    out = [0] * n
    for i in range(n):
        for j in range(n):
            k = i + j
            if k < n:
                out[k] += a[i] * b[j]
            else:
                out[k - n] -= a[i] * b[j]
    return [x % q for x in out]


def rand_poly(rng, L, N, moduli):
    return np.stack([np.array([rng.randrange(q) for _ in range(N)], dtype=np.uint64) for q in moduli[:L]])


def crt(residues, moduli):
    Q = 1
    for m in moduli:
        Q *= m
    x = 0
    for r, m in zip(residues, moduli):
        Mi = Q // m
        x += int(r) * Mi * pow(Mi, -1, m)
    return x % Q, Q


# ----------------------------------------------------------------- primes
@pytest.mark.parametrize("N,bits", [(8192, [50, 50, 55, 60]), (65536, [60] + [50] * 5 + [60] * 2), (1024, [30, 30, 40])])
def test_create_coeff_modulus(N, bits):
    mods = O.create_coeff_modulus(N, bits)
    assert len(mods) == len(bits) and len(set(mods)) == len(mods)
    for q, b in zip(mods, bits):
        assert mr_prime(q) and q.bit_length() == b and q % (2 * N) == 1
    for b in set(bits):
        got = [q for q, bb in zip(mods, bits) if bb == b]
        # The search walks down from 2^b - 2N + 1; the chosen set is exactly the
        # largest len(got) qualifying primes, handed out smallest-first
        # (src/host/modulus.cu:105-109).
        cand, v = [], (1 << b) - 2 * N + 1
        while len(cand) < len(got):
            if mr_prime(v):
                cand.append(v)
            v -= 2 * N
        assert got == sorted(cand)


def test_is_prime_matches_independent():
    rng = random.Random(5)
    for _ in range(300):
        n = rng.getrandbits(rng.choice([20, 40, 61])) | 1
        assert O.is_prime(n) == mr_prime(n)
    for p in (2, 3, 12289, 65537, 1152921504606846883):
        assert O.is_prime(p) == mr_prime(p)


def test_minimal_root_small_bruteforce():
    # q = 12289 = 3*2^12 + 1: check every x below the answer is not a primitive 2N-th root.
    q = 12289
    for N in (16, 256, 2048):
        r = O.minimal_primitive_root(2 * N, q)
        assert pow(r, N, q) == q - 1
        assert all(pow(x, N, q) != q - 1 for x in range(1, r))


def test_minimal_root_large_enumeration():
    N = 256
    q = O.create_coeff_modulus(N, [50])[0]
    r = O.minimal_primitive_root(2 * N, q)
    assert pow(r, N, q) == q - 1
    # all primitive 2N-th roots are the odd powers of any one of them
    allroots = [pow(r, k, q) for k in range(1, 2 * N, 2)]
    assert min(allroots) == r


# ----------------------------------------------------------------- NTT
def test_tables_layout():
    N = N_SMALL
    q = O.create_coeff_modulus(N, [50])[0]
    tw, tws, itw, itws, ni, nis = O.ntt_tables(N, q)
    psi = O.minimal_primitive_root(2 * N, q)
    logn = N.bit_length() - 1
    ipsi = pow(psi, -1, q)
    for i in range(N):
        assert int(tw[brv(i, logn)]) == pow(psi, i, q)
        expect = pow(ipsi, i, q)
        if brv(i, logn) == 1:
            expect = expect * pow(N, -1, q) % q  # N^-1 folded (src/host/ntt.cu:53-55)
        assert int(itw[brv(i, logn)]) == expect
        assert int(tws[i]) == (int(tw[i]) << 64) // q
        assert int(itws[i]) == (int(itw[i]) << 64) // q
    assert ni == pow(N, -1, q) and nis == (ni << 64) // q


@pytest.mark.parametrize("N,bits", [(16, [30]), (64, [50]), (256, [60])])
def test_ntt_closed_form_python(N, bits):
    """out[i] = sum_j a_j psi^((2 brv(i) + 1) j), evaluated with Python ints."""
    q = O.create_coeff_modulus(N, bits)[0]
    o = O.Oracle(N, [q, O.create_coeff_modulus(N, [bits[0] - 1])[0]], 1)
    rng = random.Random(N)
    a = [rng.randrange(q) for _ in range(N)]
    got = o.ntt_fwd(np.array([a], dtype=np.uint64))[0]
    psi = O.minimal_primitive_root(2 * N, q)
    logn = N.bit_length() - 1
    for i in range(N):
        e = 2 * brv(i, logn) + 1
        w = pow(psi, e, q)
        assert int(got[i]) == sum(a[j] * pow(w, j, q) for j in range(N)) % q


def test_ntt_naive_c_matches_fast_larger():
    N = 1024
    mods = O.create_coeff_modulus(N, [50, 60, 40])
    o = O.Oracle(N, mods, 1)
    rng = np.random.default_rng(1)
    for i, q in enumerate(mods):
        a = rng.integers(0, q, N, dtype=np.uint64)
        fast = o.ntt_fwd(a.reshape(1, N), start=i)[0]
        naive = O.ntt_naive(a, q, o.root(i))
        assert np.array_equal(fast, naive)


def test_ntt_negacyclic_convolution_and_roundtrip():
    N = 64
    mods = O.create_coeff_modulus(N, [50, 60])
    o = O.Oracle(N, mods, 1)
    rng = random.Random(3)
    for i, q in enumerate(mods):
        a = [rng.randrange(q) for _ in range(N)]
        b = [rng.randrange(q) for _ in range(N)]
        A = o.ntt_fwd(np.array([a], dtype=np.uint64), start=i)
        B = o.ntt_fwd(np.array([b], dtype=np.uint64), start=i)
        prod = np.array([[int(x) * int(y) % q for x, y in zip(A[0], B[0])]], dtype=np.uint64)
        c = o.ntt_inv(prod, start=i)[0]
        assert [int(x) for x in c] == negacyclic_mul(a, b, q)
        assert [int(x) for x in o.ntt_inv(A, start=i)[0]] == a


def test_ntt_constant_inputs_roundtrip():
    """The reference's own NTT test semantics (test/ntt_test.cu:48-50, :103-106):
    constant all-1 / all-2 inputs survive forward+inverse; NTT(1) = sum psi^((2brv(i)+1) j)."""
    N = 2048
    mods = O.create_coeff_modulus(N, [50, 50, 60])
    o = O.Oracle(N, mods, 1)
    for c in (1, 2):
        x = np.full((2, 3, N), c, dtype=np.uint64)
        f = o.ntt_fwd(x)
        assert np.array_equal(o.ntt_inv(f), x)
    # NTT of the constant polynomial c is c at every evaluation point
    x = np.zeros((1, 3, N), dtype=np.uint64)
    x[..., 0] = 7
    assert np.all(o.ntt_fwd(x) == 7)


# ----------------------------------------------------------------- chain tools
def make_chain(N, nq, alpha, qbits=50):
    bits = [60] + [qbits] * (nq - 1) + [60] * alpha
    return O.create_coeff_modulus(N, bits)


@pytest.mark.parametrize("nq,alpha,chain", [(6, 2, 1), (7, 2, 1), (5, 1, 2), (6, 3, 2)])
def test_modup_bigint(nq, alpha, chain):
    """ModUp = uncorrected fast base conversion per partition, checked with big ints."""
    N = 16
    mods = make_chain(N, nq, alpha)
    o = O.Oracle(N, mods, alpha)
    Ql = o.size_Ql(chain)
    Qmods = mods[:Ql]
    P = mods[nq:]
    rng = random.Random(nq * 10 + alpha)
    c2 = rand_poly(rng, Ql, N, mods)
    out = o.modup(chain, c2)
    beta = -(-Ql // alpha)
    assert out.shape == (beta, Ql + alpha, N)
    t = o.ntt_inv(c2)  # coefficient form, limb i uses table i
    qlp = Qmods + P
    for b in range(beta):
        st, en = b * alpha, min(b * alpha + alpha, Ql)
        part = Qmods[st:en]
        Qp = 1
        for m in part:
            Qp *= m
        assert np.array_equal(out[b, st:en], c2[st:en])
        for r in range(Ql + alpha):
            if st <= r < en:
                continue
            p = qlp[r]
            y = []
            for k in range(N):
                acc = 0
                for i, qi in enumerate(part):
                    hat = Qp // qi
                    ti = int(t[st + i, k]) * pow(hat, -1, qi) % qi
                    acc += ti * hat
                # uncorrected: acc = x + kQ with 0 <= k < |part|
                x, _ = crt([int(t[st + i, k]) for i in range(len(part))], part)
                assert (acc - x) % Qp == 0 and 0 <= (acc - x) // Qp < len(part)
                y.append(acc % p)
            row = r if r < Ql else nq + (r - Ql)
            ynt = o.ntt_fwd(np.array([y], dtype=np.uint64), start=row)[0]
            assert np.array_equal(out[b, r], ynt), (b, r)


def test_inner_product_direct():
    N, nq, alpha, chain = 16, 6, 2, 2
    mods = make_chain(N, nq, alpha)
    o = O.Oracle(N, mods, alpha)
    Ql = o.size_Ql(chain)
    beta = o.beta(chain)
    rng = np.random.default_rng(0)
    QP = len(mods)
    t = np.zeros((beta, Ql + alpha, N), dtype=np.uint64)
    key = np.zeros((o.dnum, 2, QP, N), dtype=np.uint64)
    rows = list(range(Ql)) + list(range(nq, QP))
    for r, row in enumerate(rows):
        t[:, r] = rng.integers(0, mods[row], (beta, N), dtype=np.uint64)
    for row in range(QP):
        key[:, :, row] = rng.integers(0, mods[row], (o.dnum, 2, N), dtype=np.uint64)
    cx = o.ks_inner_prod(chain, t, key)
    for k in range(2):
        for r, row in enumerate(rows):
            q = mods[row]
            exp = [sum(int(t[b, r, n]) * int(key[b, k, row, n]) for b in range(beta)) % q for n in range(N)]
            assert [int(x) for x in cx[k, r]] == exp


def test_inner_product_many_digits_bigint():
    """70 digits of residues below primes near 2^61: 65 products of such
    residues pass 2^128, so the 128-bit sums must be folded on the way
    (src/eval_key_switch.cu:175-230 folds at a threshold from the prime
    sizes).  Residues q - 1 at half the positions make every product maximal;
    checked against Python integers."""
    from gpu_util import primes_near_2_61

    N, nq, alpha, chain = 16, 70, 1, 1
    mods = primes_near_2_61(N, nq + alpha)
    o = O.Oracle(N, mods, alpha)
    Ql, beta, QP = o.size_Ql(chain), o.beta(chain), len(mods)
    assert beta == 70 and beta * (mods[-1] - 1) ** 2 >= 1 << 128
    rng = np.random.default_rng(7)
    rows = list(range(Ql)) + list(range(nq, QP))
    t = np.zeros((beta, Ql + alpha, N), dtype=np.uint64)
    key = np.zeros((o.dnum, 2, QP, N), dtype=np.uint64)
    for r, row in enumerate(rows):
        t[:, r] = rng.integers(0, mods[row], (beta, N), dtype=np.uint64)
        t[:, r, : N // 2] = mods[row] - 1
    for row in range(QP):
        key[:, :, row] = rng.integers(0, mods[row], (o.dnum, 2, N), dtype=np.uint64)
        key[:, :, row, : N // 2] = mods[row] - 1
    cx = o.ks_inner_prod(chain, t, key)
    for k in range(2):
        for r, row in enumerate(rows):
            q = mods[row]
            exp = [sum(int(t[b, r, n]) * int(key[b, k, row, n]) for b in range(beta)) % q for n in range(N)]
            assert [int(x) for x in cx[k, r]] == exp


@pytest.mark.parametrize("alpha", [1, 2, 3])
def test_moddown_exact_on_multiples_of_P(alpha):
    """ModDown(P*c extended with zero P-limbs) == c exactly."""
    N, nq, chain = 32, 5, 1
    mods = make_chain(N, nq, alpha)
    o = O.Oracle(N, mods, alpha)
    Ql = o.size_Ql(chain)
    P = 1
    for m in mods[nq:]:
        P *= m
    rng = random.Random(alpha)
    c = rand_poly(rng, Ql, N, mods)
    cx = np.zeros((Ql + alpha, N), dtype=np.uint64)
    for i in range(Ql):
        cx[i] = np.array([int(v) * (P % mods[i]) % mods[i] for v in c[i]], dtype=np.uint64)
    assert np.array_equal(o.moddown(chain, cx), c)


def test_moddown_bigint():
    N, nq, alpha, chain = 16, 5, 2, 2
    mods = make_chain(N, nq, alpha)
    o = O.Oracle(N, mods, alpha)
    Ql = o.size_Ql(chain)
    Pm = mods[nq:]
    P = Pm[0] * Pm[1]
    rng = random.Random(11)
    cx = np.zeros((Ql + alpha, N), dtype=np.uint64)
    rows = list(range(Ql)) + list(range(nq, nq + alpha))
    for r, row in enumerate(rows):
        cx[r] = [rng.randrange(mods[row]) for _ in range(N)]
    out = o.moddown(chain, cx)
    xP = np.stack([o.ntt_inv(cx[Ql + j:Ql + j + 1], start=nq + j)[0] for j in range(alpha)])
    for i in range(Ql):
        q = mods[i]
        delta = []
        for k in range(N):
            acc = 0
            for j, pj in enumerate(Pm):
                hat = P // pj
                acc += (int(xP[j, k]) * pow(hat, -1, pj) % pj) * hat
            delta.append(acc % q)
        dn = o.ntt_fwd(np.array([delta], dtype=np.uint64), start=i)[0]
        pinv = pow(P, -1, q)
        exp = [(int(cx[i, k]) - int(dn[k])) * pinv % q for k in range(N)]
        assert [int(v) for v in out[i]] == exp


@pytest.mark.parametrize("chain", [1, 2, 3])
def test_rescale_bigint_floor(chain):
    """rescale = floor((C - [C]_{q_last}) / q_last) in RNS (no rounding term)."""
    N, nq = 16, 5
    mods = make_chain(N, nq, 1)
    o = O.Oracle(N, mods, 1)
    L = o.size_Ql(chain)
    rng = random.Random(chain)
    ct = np.stack([rand_poly(rng, L, N, mods) for _ in range(2)])
    out = o.rescale(chain, ct)
    coef = np.stack([o.ntt_inv(ct[s]) for s in range(2)])
    ql = mods[L - 1]
    for s in range(2):
        exp = np.zeros((L - 1, N), dtype=object)
        for k in range(N):
            C, _ = crt([int(coef[s, i, k]) for i in range(L)], mods[:L])
            v = (C - C % ql) // ql
            for i in range(L - 1):
                exp[i, k] = v % mods[i]
        got_coef = o.ntt_inv(out[s])
        assert np.array_equal(got_coef.astype(object), exp)


def test_tensor_direct():
    N = 16
    mods = make_chain(N, 4, 1)
    o = O.Oracle(N, mods, 1)
    rng = random.Random(9)
    a = np.stack([rand_poly(rng, 4, N, mods) for _ in range(2)])
    b = np.stack([rand_poly(rng, 4, N, mods) for _ in range(2)])
    t = o.tensor(a, b)
    for l, q in enumerate(mods[:4]):
        for k in range(N):
            a0, a1, b0, b1 = (int(x[i, l, k]) for x in (a, a, b, b) for i in (0,)) if False else (
                int(a[0, l, k]), int(a[1, l, k]), int(b[0, l, k]), int(b[1, l, k]))
            assert int(t[0, l, k]) == a0 * b0 % q
            assert int(t[1, l, k]) == (a0 * b1 + a1 * b0) % q
            assert int(t[2, l, k]) == a1 * b1 % q


# ----------------------------------------------------------------- Galois
def test_elt_from_step():
    N = 1024
    m = 2 * N
    assert O.elt_from_step(0, N) == m - 1
    for s in (1, 2, 5, 100, N // 2 - 1):
        assert O.elt_from_step(s, N) == pow(5, s, m)
    for s in (1, 3, 77):
        assert O.elt_from_step(-s, N) == pow(5, N // 2 - s, m)


@pytest.mark.parametrize("step", [1, -1, 3, 0])
def test_galois_perm_is_automorphism(step):
    """NTT(a(X^elt)) == perm(NTT(a)) with a(X^elt) computed by brute force."""
    N = 64
    mods = O.create_coeff_modulus(N, [50, 60])
    o = O.Oracle(N, mods, 1)
    q = mods[0]
    elt = O.elt_from_step(step, N)
    rng = random.Random(step + 7)
    a = [rng.randrange(q) for _ in range(N)]
    sig = [0] * N
    for j, v in enumerate(a):
        k = j * elt % (2 * N)
        if k < N:
            sig[k] = (sig[k] + v) % q
        else:
            sig[k - N] = (sig[k - N] - v) % q
    A = o.ntt_fwd(np.array([a], dtype=np.uint64))
    S = o.ntt_fwd(np.array([sig], dtype=np.uint64))
    assert np.array_equal(o.apply_galois_ntt(A, elt), S)


# ----------------------------------------------------------------- scheme level
def ternary_ntt(o, rng, h):
    N = o.N
    s = np.zeros(N, dtype=np.int64)
    idx = rng.choice(N, size=h, replace=False)
    s[idx] = rng.choice([-1, 1], size=h)
    S = np.stack([(s % q).astype(np.uint64) for q in o.moduli])
    return s, o.ntt_fwd(S)


def small_err_ntt(o, rng, count):
    N = o.N
    e = rng.integers(-4, 5, (count, N))
    E = np.stack([np.stack([(ei % q).astype(np.uint64) for q in o.moduli]) for ei in e])
    return o.ntt_fwd(E)


def uniform_qp(o, rng, count):
    return np.stack([np.stack([rng.integers(0, q, o.N, dtype=np.uint64) for q in o.moduli]) for _ in range(count)])


def centered_coeffs(o, poly_ntt, L):
    """CRT-reconstruct the coefficient-domain polynomial over the first L primes, centered."""
    coef = o.ntt_inv(poly_ntt[:L])
    out = []
    for k in range(o.N):
        x, Q = crt([int(coef[i, k]) for i in range(L)], o.moduli[:L])
        out.append(x - Q if x > Q // 2 else x)
    return out


def key_decrypts_to_Ps(o, key, s_ntt, new_key):
    QP, N, alpha = o.size_QP, o.N, o.size_P
    P = 1
    for m in o.moduli[o.size_Q:]:
        P *= m
    for d in range(key.shape[0]):
        for j in range(QP):
            q = o.moduli[j]
            v = (key[d, 0, j].astype(object) + key[d, 1, j].astype(object) * s_ntt[j].astype(object)) % q
            own = d * alpha <= j < (d + 1) * alpha
            want = (P % q) * new_key[j].astype(object) % q if own else np.zeros(N, dtype=object)
            yield d, j, (v - want) % q


def test_kswitch_key_structure():
    N, nq, alpha = 32, 4, 2
    mods = make_chain(N, nq, alpha)
    o = O.Oracle(N, mods, alpha)
    rng = np.random.default_rng(4)
    _, s = ternary_ntt(o, rng, 8)
    s2 = o.mul_poly(s, s)
    a = uniform_qp(o, rng, o.dnum)
    e = small_err_ntt(o, rng, o.dnum)
    key = o.kswitch_key(s2, s, a, e)
    assert np.array_equal(key[:, 1], a)
    for d, j, resid in key_decrypts_to_Ps(o, key, s, s2):
        # key0 + key1*s - P*s2*[own] == -e  (NTT form)
        q = o.moduli[j]
        assert np.array_equal(resid.astype(np.uint64), ((-e[d, j].astype(object)) % q).astype(np.uint64))


@pytest.mark.parametrize("nq,alpha,chain", [(4, 2, 1), (5, 1, 2), (6, 3, 1)])
def test_relinearize_decrypts(nq, alpha, chain):
    """Decryption invariant: c0' + c1' s == c0 + c1 s + c2 s^2 + small noise."""
    N = 64
    mods = make_chain(N, nq, alpha)
    o = O.Oracle(N, mods, alpha)
    rng = np.random.default_rng(nq + alpha)
    _, s = ternary_ntt(o, rng, 16)
    s2 = o.mul_poly(s, s)
    rlk = o.kswitch_key(s2, s, uniform_qp(o, rng, o.dnum), small_err_ntt(o, rng, o.dnum))
    Ql = o.size_Ql(chain)
    ct3 = np.stack([np.stack([rng.integers(0, q, N, dtype=np.uint64) for q in mods[:Ql]]) for _ in range(3)])
    out = o.keyswitch(chain, ct3[:2], ct3[2], rlk)
    sQ, s2Q = s[:Ql], s2[:Ql]
    lhs = (out[0].astype(object) + out[1].astype(object) * sQ.astype(object))
    rhs = (ct3[0].astype(object) + ct3[1].astype(object) * sQ.astype(object) + ct3[2].astype(object) * s2Q.astype(object))
    qs = np.array(mods[:Ql], dtype=object)[:, None]
    diff = ((lhs - rhs) % qs).astype(np.uint64)
    noise = centered_coeffs(o, diff, Ql)
    assert max(abs(x) for x in noise) < 2 ** 30


def test_rotation_decrypts():
    N, nq, alpha, chain = 64, 4, 2, 1
    mods = make_chain(N, nq, alpha)
    o = O.Oracle(N, mods, alpha)
    rng = np.random.default_rng(21)
    _, s = ternary_ntt(o, rng, 16)
    elt = O.elt_from_step(1, N)
    s_rot = o.apply_galois_ntt(s, elt)
    glk = o.kswitch_key(s_rot, s, uniform_qp(o, rng, o.dnum), small_err_ntt(o, rng, o.dnum))
    Ql = o.size_Ql(chain)
    ct = np.stack([np.stack([rng.integers(0, q, N, dtype=np.uint64) for q in mods[:Ql]]) for _ in range(2)])
    out = o.apply_galois(chain, ct, elt, glk)
    sQ = s[:Ql].astype(object)
    qs = np.array(mods[:Ql], dtype=object)[:, None]
    dec = (out[0].astype(object) + out[1].astype(object) * sQ) % qs
    m = (ct[0].astype(object) + ct[1].astype(object) * sQ) % qs
    m_rot = o.apply_galois_ntt(m.astype(np.uint64), elt).astype(object)
    noise = centered_coeffs(o, ((dec - m_rot) % qs).astype(np.uint64), Ql)
    assert max(abs(x) for x in noise) < 2 ** 30
    # hoisted rotation decrypts to the same message (its residues differ: it
    # permutes the ModUp output instead of ModUp-ing the permuted c1)
    hr = o.hoist_rotations(chain, ct, [elt], [glk])[0]
    assert not np.array_equal(hr, out), "hoisted and plain rotation residues must differ"
    dec_h = (hr[0].astype(object) + hr[1].astype(object) * sQ) % qs
    noise = centered_coeffs(o, ((dec_h - m_rot) % qs).astype(np.uint64), Ql)
    assert max(abs(x) for x in noise) < 2 ** 30


def test_hoisting_decrypts_to_sum_of_rotations():
    """hoisting(ct, steps) decrypts to sum_e sigma_e(m) up to key-switching noise,
    and is not the sum of separately moved-down rotations (one ModDown of the sum)."""
    N, nq, alpha, chain = 64, 4, 2, 1
    mods = make_chain(N, nq, alpha)
    o = O.Oracle(N, mods, alpha)
    rng = np.random.default_rng(31)
    _, s = ternary_ntt(o, rng, 16)
    steps = [1, 2, -1]
    elts = [O.elt_from_step(t, N) for t in steps]
    keys = [o.kswitch_key(o.apply_galois_ntt(s, e), s, uniform_qp(o, rng, o.dnum), small_err_ntt(o, rng, o.dnum))
            for e in elts]
    Ql = o.size_Ql(chain)
    ct = np.stack([np.stack([rng.integers(0, q, N, dtype=np.uint64) for q in mods[:Ql]]) for _ in range(2)])
    h = o.hoisting(chain, ct, elts, keys)
    sQ = s[:Ql].astype(object)
    qs = np.array(mods[:Ql], dtype=object)[:, None]
    m = ((ct[0].astype(object) + ct[1].astype(object) * sQ) % qs).astype(np.uint64)
    want = sum(o.apply_galois_ntt(m, e).astype(object) for e in elts) % qs
    dec = (h[0].astype(object) + h[1].astype(object) * sQ) % qs
    noise = centered_coeffs(o, ((dec - want) % qs).astype(np.uint64), Ql)
    assert max(abs(x) for x in noise) < 2 ** 30
    rots = o.hoist_rotations(chain, ct, elts, keys)
    summed = sum(r.astype(object) for r in rots) % qs
    assert not np.array_equal(summed.astype(np.uint64), h)
