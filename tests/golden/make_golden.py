"""Writes the golden vectors of the CKKS hot path (tests/golden/golden_n1024.npz).

The reference ships no vectors for this path (its NTT test only round-trips
constant inputs, test/ntt_test.cu:48-50), so these are computed here, in plain
Python integers, from the definitions the reference's code implements.  This
generator shares no code with oracle/ or with the HIP library:

* primes     -- CoeffModulus::Create's rule (src/host/modulus.cu:80-111,
                src/host/numth.cu:207-233): per bit size b, primes q = 1 mod 2N
                searched downward from 2^b - 2N + 1, handed out smallest first;
                primality by deterministic Miller-Rabin.
* roots      -- the minimal primitive 2N-th root (src/host/numth.cu:309-331):
                the least g with g^N = -1 mod q, found by enumerating the odd
                powers of one such root.
* NTT        -- out[i] = sum_j a_j psi^((2 brv(i) + 1) j) mod q
                (src/ntt/ntt_1d.cu:17-76 semantics), computed as a cyclic DFT
                of the twisted sequence a_j psi^j and checked against the
                closed form evaluated term by term on one limb.
* tensor     -- (a0 b0, a0 b1 + a1 b0, a1 b1) (src/polymath.cu:463-545).
* ModUp      -- INTT, times [(Q_b/q_i)^-1]_{q_i}, uncorrected fast base
                conversion sum_i t_i [Q_b/q_i]_{p}, NTT; a digit's own limbs
                copied in NTT form (src/rns_bconv.cu:530-628).
* inner      -- cx_k[r] = sum_b modup[b][r] key[b][k][row(r)] mod p_r with
                row(r) = r for r < Ql else Q + r - Ql (src/eval_key_switch.cu:175-230).
* ModDown    -- (cx - NTT(sum_j v_j [P/p_j]_q)) [P^-1]_q with
                v_j = INTT(cx_P,j) [(P/p_j)^-1]_{p_j} (src/rns_bconv.cu:776-828).
* relinearize / multiply_and_relin -- ct_k += ModDown(cx_k) of c2
                (src/eval_key_switch.cu:294-381, src/evaluate.cu:1061-1104).
* rescale    -- [q_L^-1]_{q_j} (c_j - NTT_j(INTT_L(c_L) mod q_j)), floor
                (src/rns.cu:1128-1184).
* Galois     -- dst[i] = src[pi(i)] with slot i holding a(psi^(2 brv(i)+1)),
                so pi(i) is the slot of psi^(elt (2 brv(i)+1)); elt = 5^step
                mod 2N, step 0 -> 2N - 1 (include/galois.cuh:16-49, :98-113),
                checked against sigma(a)(X) = a(X^elt) in the coefficient domain.
* rotations  -- the reference's two orders.  apply_galois (src/evaluate.cu:
                1607-1656): c0 <- sigma(c0), c2 <- sigma(c1), then the key switch
                of c2 (ModUp of the permuted c1).  hoist_rotations (:1929-2082):
                ModUp of c1 once, then per rotation sigma on every ModUp slab
                (:2036-2045), inner product, ModDown, c0 + sigma(c0).  hoisting
                (:1732-1925): the inner products of all rotations summed mod p
                before one ModDown, plus sum_i sigma_i(c0).  The two orders give
                different residues for the same rotation (asserted here).

Run:  python tests/golden/make_golden.py   (about a minute; deterministic)
"""
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
N = 1024
LOGN = 10
SEED = 0x5EED


# ------------------------------------------------------------------ numbers
def is_prime(n):
    if n < 2:
        return False
    for p in (2, 3, 5, 7, 11, 13, 17, 19, 23, 29, 31, 37):
        if n % p == 0:
            return n == p
    d, s = n - 1, 0
    while d % 2 == 0:
        d, s = d // 2, s + 1
    for a in (2, 3, 5, 7, 11, 13, 17, 19, 23, 29, 31, 37):  # deterministic below 3.3e24
        x = pow(a, d, n)
        if x in (1, n - 1):
            continue
        for _ in range(s - 1):
            x = x * x % n
            if x == n - 1:
                break
        else:
            return False
    return True


def create_coeff_modulus(n, bits):
    """Per distinct bit size b (count c): the c largest primes q = 1 mod 2n
    below 2^b, searched from 2^b - 2n + 1 downward; the i-th request of size b
    gets the (c - 1 - i)-th found, i.e. the smallest first."""
    found = {}
    for b in sorted(set(bits)):
        need, q, got = bits.count(b), (1 << b) - 2 * n + 1, []
        while len(got) < need:
            if is_prime(q):
                got.append(q)
            q -= 2 * n
        found[b] = got
    used = {b: 0 for b in found}
    out = []
    for b in bits:
        out.append(found[b][len(found[b]) - 1 - used[b]])
        used[b] += 1
    return out


def minimal_root(q, n=N):
    m = 2 * n
    for x in range(2, q):
        g = pow(x, (q - 1) // m, q)
        if pow(g, n, q) == q - 1:
            break
    best, g2, cur = g, g * g % q, g
    for _ in range(n - 1):
        cur = cur * g2 % q
        best = min(best, cur)
    return best


def brv(x, bits=LOGN):
    return int(format(x, f"0{bits}b")[::-1], 2)


# ------------------------------------------------------------------ transforms
def dft_brv(a, w, q):
    """y[i] = sum_j a_j w^(brv(i) j): iterative radix-2 DIT on bit-reversed input
    yields natural order; y is then re-indexed by brv."""
    n = len(a)
    x = [a[brv(i)] for i in range(n)]
    m = 1
    while m < n:
        wm = pow(w, n // (2 * m), q)
        for k in range(0, n, 2 * m):
            wk = 1
            for j in range(m):
                t = wk * x[k + j + m] % q
                u = x[k + j]
                x[k + j], x[k + j + m] = (u + t) % q, (u - t) % q
                wk = wk * wm % q
        m *= 2
    return [x[brv(i)] for i in range(n)]


def ntt(a, q, psi):
    return dft_brv([int(v) * pow(psi, j, q) % q for j, v in enumerate(a)], psi * psi % q, q)


def intt(y, q, psi):
    n = len(y)
    ipsi, ninv = pow(psi, -1, q), pow(n, -1, q)
    # a_j psi^j = N^-1 sum_m Y_m w^(-m j) with Y_m = y[brv(m)] the natural-order DFT
    z = dft_brv([int(y[brv(m)]) for m in range(n)], pow(psi * psi % q, -1, q), q)
    return [z[brv(j)] * ninv % q * pow(ipsi, j, q) % q for j in range(n)]


def ntt_closed_form(a, q, psi):
    n = len(a)
    return [sum(int(a[j]) * pow(psi, (2 * brv(i) + 1) * j, q) for j in range(n)) % q for i in range(n)]


class Chain:
    def __init__(self, moduli, alpha):
        self.mods = list(moduli)
        self.P = alpha
        self.Q = len(moduli) - alpha
        self.psi = [minimal_root(q) for q in moduli]

    def ntt(self, a, row):
        return ntt(a, self.mods[row], self.psi[row])

    def intt(self, a, row):
        return intt(a, self.mods[row], self.psi[row])


def modup(ch, c2):
    Ql, a = len(c2), ch.P
    rows = list(range(Ql)) + [ch.Q + j for j in range(a)]
    t = [ch.intt(c2[i], i) for i in range(Ql)]
    beta = -(-Ql // a)
    out = []
    for b in range(beta):
        I = list(range(b * a, min((b + 1) * a, Ql)))
        Qb = 1
        for i in I:
            Qb *= ch.mods[i]
        u = {i: [v * pow(Qb // ch.mods[i], -1, ch.mods[i]) % ch.mods[i] for v in t[i]] for i in I}
        slab = []
        for r, row in enumerate(rows):
            if r in I:
                slab.append([int(v) for v in c2[r]])
                continue
            p = ch.mods[row]
            y = [sum(u[i][x] * (Qb // ch.mods[i] % p) for i in I) % p for x in range(N)]
            slab.append(ch.ntt(y, row))
        out.append(slab)
    return out


def inner(ch, slabs, key, Ql):
    QlP = Ql + ch.P
    cx = []
    for k in range(2):
        polys = []
        for r in range(QlP):
            row = r if r < Ql else ch.Q + r - Ql
            p = ch.mods[row]
            polys.append([sum(slabs[b][r][x] * int(key[b][k][row][x]) for b in range(len(slabs))) % p
                          for x in range(N)])
        cx.append(polys)
    return cx


def moddown(ch, cxk, Ql):
    a = ch.P
    Pp = 1
    for j in range(a):
        Pp *= ch.mods[ch.Q + j]
    v = []
    for j in range(a):
        pj = ch.mods[ch.Q + j]
        s = pow(Pp // pj, -1, pj)
        v.append([x * s % pj for x in ch.intt(cxk[Ql + j], ch.Q + j)])
    out = []
    for i in range(Ql):
        q = ch.mods[i]
        d = [sum(v[j][x] * (Pp // ch.mods[ch.Q + j] % q) for j in range(a)) % q for x in range(N)]
        dn = ch.ntt(d, i)
        pinv = pow(Pp % q, -1, q)
        out.append([(int(cxk[i][x]) - dn[x]) * pinv % q for x in range(N)])
    return out


def rescale(ch, ct):
    L = len(ct[0])
    ql = ch.mods[L - 1]
    out = []
    for poly in ct:
        last = ch.intt(poly[L - 1], L - 1)
        res = []
        for j in range(L - 1):
            q = ch.mods[j]
            dn = ch.ntt([v % q for v in last], j)
            inv = pow(ql, -1, q)
            res.append([(int(poly[j][x]) - dn[x]) * inv % q for x in range(N)])
        out.append(res)
    return out


def elt_from_step(step):
    m = 2 * N
    return m - 1 if step == 0 else pow(5, step % (N // 2), m)


def galois_perm(elt):
    slot = {2 * brv(i) + 1: i for i in range(N)}  # odd exponent -> NTT slot
    return [slot[elt * (2 * brv(i) + 1) % (2 * N)] for i in range(N)]


def permute(poly_limbs, pm):
    return [[int(limb[pm[i]]) for i in range(N)] for limb in poly_limbs]


def add_limbs(a, b, mods):
    return [[(u + v) % q for u, v in zip(x, y)] for x, y, q in zip(a, b, mods)]


def ksw_out(ch, c0, cx, Ql):
    """(c0 + ModDown(cx_0), ModDown(cx_1)): keyswitch_inplace on (c0, 0)."""
    md = [moddown(ch, cx[k], Ql) for k in range(2)]
    return [add_limbs(c0, md[0], ch.mods[:Ql]), md[1]]


def apply_galois_ct(ch, ct, elt, key):
    Ql = len(ct[0])
    pm = galois_perm(elt)
    c0, c1 = permute(ct[0], pm), permute(ct[1], pm)
    return ksw_out(ch, c0, inner(ch, modup(ch, c1), key, Ql), Ql)


def qlp_mods(ch, Ql):
    return [ch.mods[r] for r in range(Ql)] + [ch.mods[ch.Q + j] for j in range(ch.P)]


def hoist_rotations_ct(ch, ct, elts, keys):
    Ql = len(ct[0])
    slabs = modup(ch, [[int(v) for v in limb] for limb in ct[1]])
    out = []
    for elt, key in zip(elts, keys):
        pm = galois_perm(elt)
        rot = [permute(slab, pm) for slab in slabs]
        out.append(ksw_out(ch, permute(ct[0], pm), inner(ch, rot, key, Ql), Ql))
    return out


def hoisting_ct(ch, ct, elts, keys):
    Ql = len(ct[0])
    slabs = modup(ch, [[int(v) for v in limb] for limb in ct[1]])
    acc0, acc = None, None
    for elt, key in zip(elts, keys):
        pm = galois_perm(elt)
        c0 = permute(ct[0], pm)
        cx = inner(ch, [permute(slab, pm) for slab in slabs], key, Ql)
        acc0 = c0 if acc0 is None else add_limbs(acc0, c0, ch.mods[:Ql])
        acc = cx if acc is None else [add_limbs(acc[k], cx[k], qlp_mods(ch, Ql)) for k in range(2)]
    return ksw_out(ch, acc0, acc, Ql)


def uniform(rng, shape, mods):
    """uint64 residues, limb axis -2 over `mods`."""
    *pre, L, n = shape
    out = np.empty(shape, dtype=np.uint64)
    for l in range(L):
        out[..., l, :] = rng.integers(0, mods[l], size=tuple(pre) + (n,), dtype=np.uint64)
    return out


def u64(x):
    return np.array(x, dtype=np.uint64)


def main():
    rng = np.random.default_rng(SEED)
    g = {}
    # --- config-1 primes at the config-1 degree, and the large configs' chains
    chains = {
        "c1_n8192": (8192, [50, 50, 55, 60]),
        "c2_n65536": (65536, [50] * 35 + [60]),
        "c3_n65536": (65536, [60] + [50] * 23 + [60] * 4),
        "c4_n65536": (65536, [60] + [40] * 19 + [60] * 4),
    }
    for name, (n, bits) in chains.items():
        g[f"primes_{name}"] = u64(create_coeff_modulus(n, bits))
    c1 = [int(q) for q in g["primes_c1_n8192"]]
    g["roots_c1_n8192"] = u64([minimal_root(q, 8192) for q in c1])

    # --- NTT at N = 1024 over config-1 bit sizes
    ntt_mods = create_coeff_modulus(N, [50, 50, 55, 60])
    ntt_psi = [minimal_root(q) for q in ntt_mods]
    x = uniform(rng, (4, N), ntt_mods)
    y = u64([ntt([int(v) for v in x[l]], ntt_mods[l], ntt_psi[l]) for l in range(4)])
    assert [int(v) for v in y[0]] == ntt_closed_form(x[0], ntt_mods[0], ntt_psi[0])
    assert all([int(v) for v in x[l]] == intt([int(v) for v in y[l]], ntt_mods[l], ntt_psi[l]) for l in range(4))
    g.update(ntt_moduli=u64(ntt_mods), ntt_roots=u64(ntt_psi), ntt_in=x, ntt_out=y)

    # --- Galois permutations
    steps = [1, 2, 7, N // 2 - 1, 0]
    elts = [elt_from_step(s) for s in steps]
    perms = [galois_perm(e) for e in elts]
    # sigma(a)(X) = a(X^elt) in the coefficient domain, then NTT, equals the permuted NTT
    a = [int(v) for v in x[0]]
    q, psi = ntt_mods[0], ntt_psi[0]
    for e, pm in zip(elts[:2] + elts[-1:], perms[:2] + perms[-1:]):
        s = [0] * N
        for j, v in enumerate(a):
            k = j * e % (2 * N)
            if k < N:
                s[k] = (s[k] + v) % q
            else:
                s[k - N] = (s[k - N] - v) % q
        A = ntt(a, q, psi)
        assert ntt(s, q, psi) == [A[pm[i]] for i in range(N)]
    g.update(galois_steps=np.array(steps, dtype=np.int64), galois_elts=u64(elts),
             galois_perms=np.array(perms, dtype=np.uint32))

    # --- key switching on the chain {60, 50, 50, 50 | 60, 60}: |Q| = 4, alpha = 2, dnum = 2
    ks_mods = create_coeff_modulus(N, [60, 50, 50, 50, 60, 60])
    ch = Chain(ks_mods, 2)
    Q, QP = 4, 6
    a_ct = uniform(rng, (2, Q, N), ks_mods)
    b_ct = uniform(rng, (2, Q, N), ks_mods)
    key = np.stack([uniform(rng, (2, QP, N), ks_mods) for _ in range(2)])  # [dnum][2][QP][N]
    d = []
    for l in range(Q):
        q = ks_mods[l]
        a0, a1 = [int(v) for v in a_ct[0][l]], [int(v) for v in a_ct[1][l]]
        b0, b1 = [int(v) for v in b_ct[0][l]], [int(v) for v in b_ct[1][l]]
        d.append(([u * v % q for u, v in zip(a0, b0)],
                  [(u * v + s * t) % q for u, v, s, t in zip(a0, b1, a1, b0)],
                  [u * v % q for u, v in zip(a1, b1)]))
    tensor = u64([[d[l][k] for l in range(Q)] for k in range(3)])  # [3][Q][N]
    c2 = [[int(v) for v in tensor[2][l]] for l in range(Q)]
    slabs = modup(ch, c2)
    cx = inner(ch, slabs, key, Q)
    md = [moddown(ch, cx[k], Q) for k in range(2)]
    relin = u64([[[(int(tensor[k][l][x]) + md[k][l][x]) % ks_mods[l] for x in range(N)] for l in range(Q)]
                 for k in range(2)])
    resc = u64(rescale(ch, [[list(map(int, relin[k][l])) for l in range(Q)] for k in range(2)]))
    # a lower level (chain index 2: Ql = 3, beta = 2 with a short last digit)
    c2_low = uniform(rng, (3, N), ks_mods)
    slabs_low = modup(ch, [[int(v) for v in c2_low[l]] for l in range(3)])
    g.update(ks_moduli=u64(ks_mods), ks_roots=u64(ch.psi), ks_alpha=np.array(2), ks_a=a_ct, ks_b=b_ct,
             ks_key=key, ks_tensor=tensor, ks_modup=u64(slabs), ks_cx=u64(cx), ks_moddown=u64(md),
             ks_mul_relin=relin, ks_rescale=resc, ks_c2_low=c2_low, ks_modup_low=u64(slabs_low))
    # --- rotations: apply_galois (permute, then key-switch) against the hoisted
    # forms (ModUp, then permute the slabs), on fresh random keys per element
    rot_ct = uniform(rng, (2, Q, N), ks_mods)
    rot_steps = [1, 0]
    rot_elts = [elt_from_step(t) for t in rot_steps]
    rot_keys = np.stack([np.stack([uniform(rng, (2, QP, N), ks_mods) for _ in range(2)]) for _ in rot_elts])
    ct_int = [[[int(v) for v in limb] for limb in poly] for poly in rot_ct]
    ag = u64(apply_galois_ct(ch, ct_int, rot_elts[0], rot_keys[0]))
    hr = u64(hoist_rotations_ct(ch, ct_int, rot_elts, rot_keys))
    assert not np.array_equal(ag, hr[0]), "the two rotation orders must give different residues"
    # hoisting at chain index 2 (Ql = 3: a short last digit and the P-row remap)
    h_ct = uniform(rng, (2, 3, N), ks_mods)
    h_steps = [1, 2]
    h_elts = [elt_from_step(t) for t in h_steps]
    h_keys = np.stack([np.stack([uniform(rng, (2, QP, N), ks_mods) for _ in range(2)]) for _ in h_elts])
    hs = u64(hoisting_ct(ch, [[[int(v) for v in limb] for limb in poly] for poly in h_ct], h_elts, h_keys))
    g.update(rot_ct=rot_ct, rot_steps=np.array(rot_steps, dtype=np.int64), rot_elts=u64(rot_elts),
             rot_keys=rot_keys, rot_apply_galois=ag, rot_hoist_rotations=hr, hoisting_ct=h_ct,
             hoisting_elts=u64(h_elts), hoisting_keys=h_keys, hoisting_out=hs)
    np.savez(os.path.join(HERE, "golden_n1024.npz"), **g)
    print("wrote", os.path.join(HERE, "golden_n1024.npz"), sorted(g))


if __name__ == "__main__":
    main()
