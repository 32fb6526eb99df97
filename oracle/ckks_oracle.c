/*
 * CPU oracle for the CKKS evaluation hot path -- TEST INFRASTRUCTURE ONLY.
 *
 * Restates the reference's (gold9598/phantom-fhe) arithmetic in plain C from
 * the mathematics.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg load this library; the HIP product never does.
 *
 * Every output is a canonical residue in [0, q).  The reference's device
 * reductions (Shoup with a final csub, Barrett-128 with a single csub on
 * inputs < 2^126) are exact, so canonical residues of the same formulas are
 * bit-identical to what the reference computes.
 *
 * Parity pinning of each function lives in tests/test_oracle.py (closed
 * forms, brute force, big-integer CRT identities) and tests/test_golden.py
 * (vectors computed independently in plain Python integers).
 */
#include "ckks_oracle.h"

#include <stdlib.h>
#include <string.h>

typedef unsigned __int128 u128;

/* ------------------------------------------------------------------------ */
/* scalar modular arithmetic                                                 */
/* ------------------------------------------------------------------------ */

uint64_t orc_mulmod(uint64_t a, uint64_t b, uint64_t q) { return (uint64_t)(((u128)a * b) % q); }

uint64_t orc_powmod(uint64_t a, uint64_t e, uint64_t q) {
    uint64_t r = 1 % q;
    a %= q;
    while (e) {
        if (e & 1) r = orc_mulmod(r, a, q);
        a = orc_mulmod(a, a, q);
        e >>= 1;
    }
    return r;
}

/* inverse modulo a prime (Fermat); callers only pass prime moduli */
uint64_t orc_invmod(uint64_t a, uint64_t q) { return orc_powmod(a % q, q - 2, q); }

/* compute_shoup: floor(w * 2^64 / q) (include/host/uintarithsmallmod.h:119-124) */
uint64_t orc_shoup(uint64_t w, uint64_t q) { return (uint64_t)(((u128)w << 64) / q); }

/* multiply_uint_mod_shoup (include/host/uintarithsmallmod.h:131-138): exact
 * for any y < 2^64 when w < q < 2^63; returns the canonical residue. */
static inline uint64_t mul_shoup(uint64_t y, uint64_t w, uint64_t ws, uint64_t q) {
    uint64_t hi = (uint64_t)(((u128)y * ws) >> 64);
    uint64_t r = y * w - hi * q;
    return r >= q ? r - q : r;
}

static inline uint64_t add_mod(uint64_t a, uint64_t b, uint64_t q) {
    uint64_t r = a + b;
    return r >= q ? r - q : r;
}

static inline uint64_t sub_mod(uint64_t a, uint64_t b, uint64_t q) { return a >= b ? a - b : a + q - b; }

static uint32_t brv(uint32_t x, int bits) {
    uint32_t r = 0;
    for (int i = 0; i < bits; i++) r |= ((x >> i) & 1u) << (bits - 1 - i);
    return r;
}

static int ilog2(uint64_t n) {
    int r = 0;
    while ((1ULL << r) < n) r++;
    return r;
}

/* ------------------------------------------------------------------------ */
/* primes (src/host/numth.cu:129-233, src/host/modulus.cu:80-111)            */
/* ------------------------------------------------------------------------ */

/* Deterministic Miller-Rabin (exact for n < 3.3e24).  The reference runs
 * trial division by 2..13 plus 40 Miller-Rabin rounds (numth.cu:129-205);
 * both decide primality, this one without randomness. */
int orc_is_prime(uint64_t n) {
    static const uint64_t small[] = {2, 3, 5, 7, 11, 13, 17, 19, 23, 29, 31, 37};
    if (n < 2) return 0;
    for (size_t i = 0; i < sizeof(small) / sizeof(small[0]); i++) {
        if (n == small[i]) return 1;
        if (n % small[i] == 0) return 0;
    }
    uint64_t d = n - 1;
    int r = 0;
    while ((d & 1) == 0) {
        d >>= 1;
        r++;
    }
    for (size_t i = 0; i < sizeof(small) / sizeof(small[0]); i++) {
        uint64_t x = orc_powmod(small[i], d, n);
        if (x == 1 || x == n - 1) continue;
        int ok = 0;
        for (int k = 1; k < r; k++) {
            x = orc_mulmod(x, x, n);
            if (x == n - 1) {
                ok = 1;
                break;
            }
        }
        if (!ok) return 0;
    }
    return 1;
}

/* get_primes (numth.cu:207-233): walk down from 2^b - 2N + 1 in steps of 2N,
 * collecting `count` primes above 2^(b-1).  Result is largest-first. */
static int get_primes(uint64_t N, int bits, size_t count, uint64_t *dst) {
    uint64_t factor = 2 * N;
    uint64_t value = (1ULL << bits) - factor + 1;
    uint64_t lower = 1ULL << (bits - 1);
    size_t found = 0;
    while (found < count && value > lower) {
        if (orc_is_prime(value)) dst[found++] = value;
        value -= factor;
    }
    return found == count ? 0 : -1;
}

/* CoeffModulus::Create (modulus.cu:80-111): per bit size, the primes found are
 * consumed from the back, so the first request of a size gets the smallest of
 * the `count` primes found and later requests get larger ones. */
int orc_create_coeff_modulus(uint64_t N, const int *bit_sizes, size_t count, uint64_t *out) {
    for (size_t i = 0; i < count; i++) {
        int b = bit_sizes[i];
        if (b < 2 || b > 60) return -1;
    }
    for (size_t i = 0; i < count; i++) {
        int b = bit_sizes[i];
        size_t same = 0, rank = 0;
        for (size_t j = 0; j < count; j++) {
            if (bit_sizes[j] == b) {
                if (j < i) rank++;
                same++;
            }
        }
        uint64_t *tmp = (uint64_t *)malloc(same * sizeof(uint64_t));
        if (get_primes(N, b, same, tmp) != 0) {
            free(tmp);
            return -1;
        }
        out[i] = tmp[same - 1 - rank];
        free(tmp);
    }
    return 0;
}

/* try_minimal_primitive_root (numth.cu:309-331): the smallest primitive
 * degree-th root of unity mod q.  The reference starts from a random
 * primitive root g and scans g, g^3, g^5, ... (all primitive roots); the
 * minimum over that set does not depend on g.  Here g is found
 * deterministically. */
uint64_t orc_minimal_primitive_root(uint64_t degree, uint64_t q) {
    if ((q - 1) % degree != 0) return 0;
    uint64_t cof = (q - 1) / degree;
    uint64_t g = 0;
    for (uint64_t x = 2; x < q; x++) {
        uint64_t c = orc_powmod(x, cof, q);
        if (orc_powmod(c, degree / 2, q) == q - 1) {
            g = c;
            break;
        }
    }
    if (!g) return 0;
    uint64_t g2 = orc_mulmod(g, g, q);
    uint64_t cur = g, best = g;
    for (uint64_t i = 0; i < degree / 2; i++) {
        if (cur < best) best = cur;
        cur = orc_mulmod(cur, g2, q);
    }
    return best;
}

/* ------------------------------------------------------------------------ */
/* NTT tables and transforms                                                 */
/* ------------------------------------------------------------------------ */

/* arith::NTT::NTT (src/host/ntt.cu:11-56):
 *   tw[brv(i)]  = psi^i,  itw[brv(i)] = psi^-i,  then itw[1] *= N^-1. */
void orc_ntt_tables(uint64_t N, uint64_t q, uint64_t *tw, uint64_t *tw_shoup, uint64_t *itw,
                    uint64_t *itw_shoup, uint64_t *ninv, uint64_t *ninv_shoup) {
    int logn = ilog2(N);
    uint64_t psi = orc_minimal_primitive_root(2 * N, q);
    uint64_t ipsi = orc_invmod(psi, q);
    uint64_t p = 1, ip = 1;
    for (uint64_t i = 0; i < N; i++) {
        uint32_t r = brv((uint32_t)i, logn);
        tw[r] = p;
        itw[r] = ip;
        p = orc_mulmod(p, psi, q);
        ip = orc_mulmod(ip, ipsi, q);
    }
    uint64_t ni = orc_invmod(N % q, q);
    itw[1] = orc_mulmod(itw[1], ni, q);
    for (uint64_t i = 0; i < N; i++) {
        tw_shoup[i] = orc_shoup(tw[i], q);
        itw_shoup[i] = orc_shoup(itw[i], q);
    }
    *ninv = ni;
    *ninv_shoup = orc_shoup(ni, q);
}

/* Forward negacyclic NTT, radix-2 Cooley-Tukey in the order of
 * inplace_fnwt_radix2 (src/ntt/ntt_1d.cu:17-76): stage m uses tw[m + i], with
 * its precomputed Shoup quotient tws[m + i] (the reference's tables carry the
 * same pairs, include/ntt.cuh:34-129).  Butterflies are Harvey's lazy form, as
 * the reference's (include/butterfly.cuh:17-76): operands stay in [0, 4q)
 * between stages (q < 2^62) and one correction at the end makes them
 * canonical, so the output equals the textbook transform's. */
void orc_ntt_fwd_limb(uint64_t *a, uint64_t N, uint64_t q, const uint64_t *tw, const uint64_t *tws) {
    const uint64_t q2 = 2 * q;
    for (uint64_t m = 1, t = N >> 1; m < N; m <<= 1, t >>= 1) {
        for (uint64_t i = 0; i < m; i++) {
            const uint64_t w = tw[m + i], ws = tws[m + i];
            uint64_t *restrict x = a + 2 * i * t, *restrict y = x + t;
            for (uint64_t j = 0; j < t; j++) {
                uint64_t u = x[j];
                u = u >= q2 ? u - q2 : u;                                   /* [0, 2q) */
                const uint64_t v = y[j] * w - (uint64_t)(((u128)y[j] * ws) >> 64) * q; /* [0, 2q) */
                x[j] = u + v;
                y[j] = u - v + q2;
            }
        }
    }
    for (uint64_t j = 0; j < N; j++) {
        uint64_t u = a[j];
        u = u >= q2 ? u - q2 : u;
        a[j] = u >= q ? u - q : u;
    }
}

/* Inverse, Gentleman-Sande in the order of inplace_inwt_radix2
 * (src/ntt/ntt_1d.cu:180-240): stage m uses itw[m + i]; in the last stage the
 * sum half is scaled by N^-1 and the difference half gets N^-1 through the
 * folded itw[1].  Lazy as the reference's (include/butterfly.cuh:78-134):
 * operands in [0, 2q) between stages, canonical at the end. */
void orc_ntt_inv_limb(uint64_t *a, uint64_t N, uint64_t q, const uint64_t *itw, const uint64_t *itws,
                      uint64_t ninv) {
    const uint64_t q2 = 2 * q, ninv_s = orc_shoup(ninv, q);
    for (uint64_t m = N >> 1, t = 1; m >= 1; m >>= 1, t <<= 1) {
        for (uint64_t i = 0; i < m; i++) {
            const uint64_t w = itw[m + i], ws = itws[m + i];
            uint64_t *restrict x = a + 2 * i * t, *restrict y = x + t;
            for (uint64_t j = 0; j < t; j++) {
                const uint64_t u = x[j], v = y[j];
                uint64_t s = u + v;
                s = s >= q2 ? s - q2 : s;                                    /* [0, 2q) */
                const uint64_t d = u - v + q2;                               /* [0, 4q) */
                if (m == 1) s = s * ninv - (uint64_t)(((u128)s * ninv_s) >> 64) * q;
                x[j] = s;
                y[j] = d * w - (uint64_t)(((u128)d * ws) >> 64) * q;         /* [0, 2q) */
            }
        }
        if (m == 1) break;
    }
    for (uint64_t j = 0; j < N; j++) a[j] = a[j] >= q ? a[j] - q : a[j];
}

void orc_ntt_naive_limb(const uint64_t *a, uint64_t *out, uint64_t N, uint64_t q, uint64_t psi) {
    int logn = ilog2(N);
    for (uint64_t i = 0; i < N; i++) {
        uint64_t e = 2 * (uint64_t)brv((uint32_t)i, logn) + 1;
        uint64_t root = orc_powmod(psi, e, q);
        uint64_t acc = 0, p = 1;
        for (uint64_t j = 0; j < N; j++) {
            acc = add_mod(acc, orc_mulmod(a[j], p, q), q);
            p = orc_mulmod(p, root, q);
        }
        out[i] = acc;
    }
}

/* ------------------------------------------------------------------------ */
/* context                                                                   */
/* ------------------------------------------------------------------------ */

struct orc_ctx {
    uint64_t N;
    int logN;
    size_t size_QP, size_P, size_Q;
    uint64_t *moduli;
    uint64_t *roots;
    uint64_t *tw, *tws, *itw, *itws; /* [size_QP][N] */
    uint64_t *ninv, *ninvs;
};

orc_ctx *orc_ctx_create(uint64_t N, const uint64_t *moduli, size_t size_QP, size_t size_P) {
    orc_ctx *c = (orc_ctx *)calloc(1, sizeof(orc_ctx));
    c->N = N;
    c->logN = ilog2(N);
    c->size_QP = size_QP;
    c->size_P = size_P;
    c->size_Q = size_QP - size_P;
    c->moduli = (uint64_t *)malloc(size_QP * sizeof(uint64_t));
    memcpy(c->moduli, moduli, size_QP * sizeof(uint64_t));
    c->roots = (uint64_t *)malloc(size_QP * sizeof(uint64_t));
    c->tw = (uint64_t *)malloc(size_QP * N * sizeof(uint64_t));
    c->tws = (uint64_t *)malloc(size_QP * N * sizeof(uint64_t));
    c->itw = (uint64_t *)malloc(size_QP * N * sizeof(uint64_t));
    c->itws = (uint64_t *)malloc(size_QP * N * sizeof(uint64_t));
    c->ninv = (uint64_t *)malloc(size_QP * sizeof(uint64_t));
    c->ninvs = (uint64_t *)malloc(size_QP * sizeof(uint64_t));
    for (size_t i = 0; i < size_QP; i++) {
        c->roots[i] = orc_minimal_primitive_root(2 * N, moduli[i]);
        orc_ntt_tables(N, moduli[i], c->tw + i * N, c->tws + i * N, c->itw + i * N, c->itws + i * N,
                       &c->ninv[i], &c->ninvs[i]);
    }
    return c;
}

void orc_ctx_destroy(orc_ctx *c) {
    if (!c) return;
    free(c->moduli);
    free(c->roots);
    free(c->tw);
    free(c->tws);
    free(c->itw);
    free(c->itws);
    free(c->ninv);
    free(c->ninvs);
    free(c);
}

size_t orc_ctx_size_QP(const orc_ctx *c) { return c->size_QP; }

#ifndef ORC_BUILD_FLAGS
#define ORC_BUILD_FLAGS "unknown flags"
#endif
/* Compiler and flags this library was built with (reported beside CPU timings). */
const char *orc_build_info(void) {
#ifdef __VERSION__
    return "cc " __VERSION__ ", " ORC_BUILD_FLAGS;
#else
    return ORC_BUILD_FLAGS;
#endif
}
uint64_t orc_ctx_root(const orc_ctx *c, size_t i) { return c->roots[i]; }

const uint64_t *orc_ctx_table(const orc_ctx *c, size_t i, int which) {
    switch (which) {
    case 0: return c->tw + i * c->N;
    case 1: return c->tws + i * c->N;
    case 2: return c->itw + i * c->N;
    case 3: return c->itws + i * c->N;
    case 4: return c->ninv + i;
    case 5: return c->ninvs + i;
    default: return 0;
    }
}

static void fwd_limb(const orc_ctx *c, uint64_t *a, size_t tidx) {
    orc_ntt_fwd_limb(a, c->N, c->moduli[tidx], c->tw + tidx * c->N, c->tws + tidx * c->N);
}

static void inv_limb(const orc_ctx *c, uint64_t *a, size_t tidx) {
    orc_ntt_inv_limb(a, c->N, c->moduli[tidx], c->itw + tidx * c->N, c->itws + tidx * c->N, c->ninv[tidx]);
}

void orc_ntt_fwd(const orc_ctx *c, uint64_t *data, size_t M, size_t L, size_t start, int threads) {
    long total = (long)(M * L);
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
    for (long k = 0; k < total; k++) fwd_limb(c, data + (size_t)k * c->N, start + (size_t)k % L);
}

void orc_ntt_inv(const orc_ctx *c, uint64_t *data, size_t M, size_t L, size_t start, int threads) {
    long total = (long)(M * L);
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
    for (long k = 0; k < total; k++) inv_limb(c, data + (size_t)k * c->N, start + (size_t)k % L);
}

/* ------------------------------------------------------------------------ */
/* tensor product (src/polymath.cu:463-532)                                  */
/* ------------------------------------------------------------------------ */

void orc_tensor(const orc_ctx *c, size_t L, const uint64_t *a, const uint64_t *b, uint64_t *out) {
    size_t N = c->N, LN = L * N;
    for (size_t l = 0; l < L; l++) {
        uint64_t q = c->moduli[l];
        for (size_t k = 0; k < N; k++) {
            size_t t = l * N + k;
            uint64_t a0 = a[t], a1 = a[t + LN], b0 = b[t], b1 = b[t + LN];
            out[t] = orc_mulmod(a0, b0, q);
            out[t + LN] = add_mod(orc_mulmod(a0, b1, q), orc_mulmod(a1, b0, q), q);
            out[t + 2 * LN] = orc_mulmod(a1, b1, q);
        }
    }
}

void orc_tensor_square(const orc_ctx *c, size_t L, const uint64_t *a, uint64_t *out) {
    orc_tensor(c, L, a, a, out);
}

void orc_mul_poly(const orc_ctx *c, size_t L, size_t start, const uint64_t *a, const uint64_t *b, uint64_t *out) {
    size_t N = c->N;
    for (size_t l = 0; l < L; l++) {
        uint64_t q = c->moduli[start + l];
        for (size_t k = 0; k < N; k++) out[l * N + k] = orc_mulmod(a[l * N + k], b[l * N + k], q);
    }
}

/* ------------------------------------------------------------------------ */
/* RNS tools at a chain index (src/rns.cu:11-195)                            */
/* ------------------------------------------------------------------------ */

/* chain_index c in [1, |Q|] holds |Ql| = |Q| - (c - 1) primes (src/context.cu:145-159) */
static size_t size_Ql(const orc_ctx *c, size_t chain_index) { return c->size_Q - (chain_index - 1); }

/* table row of position r in the QlP basis: Ql primes, then P primes at the
 * tail of the QP table (src/eval_key_switch.cu:182, src/ntt/fntt_2d.cu:441-443) */
static size_t qlp_row(const orc_ctx *c, size_t Ql, size_t r) { return r < Ql ? r : c->size_Q + (r - Ql); }

size_t orc_beta(const orc_ctx *c, size_t chain_index) {
    size_t Ql = size_Ql(c, chain_index), a = c->size_P;
    return (Ql + a - 1) / a;
}

size_t orc_dnum(const orc_ctx *c) { return c->size_P ? c->size_Q / c->size_P : 0; }

/* punctured product prod_{k in set, k != skip} m_k  mod  p */
static uint64_t punctured_mod(const uint64_t *m, size_t n, size_t skip, uint64_t p) {
    uint64_t r = 1 % p;
    for (size_t k = 0; k < n; k++)
        if (k != skip) r = orc_mulmod(r, m[k] % p, p);
    return r;
}

/* ModUp (src/rns_bconv.cu:530-628, precompute src/rns.cu:141-190).
 *   t_i = INTT(c2_i) * [(Q_part/q_i)^-1]_{q_i}             (coefficient form)
 *   slab b, own limbs  : copy of c2 (NTT form)
 *   slab b, other limbs: NTT( sum_{i in part b} t_i * [Q_part/q_i]_{p_j} mod p_j )
 * For alpha == 1 the partition holds one prime and the formula reduces to
 * t mod p_j (modup_bconv_single_p_kernel, src/rns_bconv.cu:432-453). */
void orc_modup(const orc_ctx *c, size_t chain_index, const uint64_t *c2, uint64_t *t_mod_up, int threads) {
    size_t N = c->N, alpha = c->size_P, Ql = size_Ql(c, chain_index), QlP = Ql + alpha;
    size_t beta = (Ql + alpha - 1) / alpha;
    uint64_t *t = (uint64_t *)malloc(Ql * N * sizeof(uint64_t));
    memcpy(t, c2, Ql * N * sizeof(uint64_t));
    for (size_t i = 0; i < Ql; i++) {
        inv_limb(c, t + i * N, i);
        size_t b = i / alpha, st = b * alpha, sz = (b == beta - 1) ? Ql - alpha * (beta - 1) : alpha;
        uint64_t q = c->moduli[i];
        uint64_t hat = punctured_mod(c->moduli + st, sz, i - st, q);
        uint64_t hinv = orc_invmod(hat, q), hs = orc_shoup(hinv, q);
        for (size_t k = 0; k < N; k++) t[i * N + k] = mul_shoup(t[i * N + k], hinv, hs, q);
    }
    for (size_t b = 0; b < beta; b++) {
        size_t st = b * alpha, sz = (b == beta - 1) ? Ql - alpha * (beta - 1) : alpha, en = st + sz;
        uint64_t *slab = t_mod_up + b * QlP * N;
        memcpy(slab + st * N, c2 + st * N, sz * N * sizeof(uint64_t));
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
        for (long rr = 0; rr < (long)QlP; rr++) {
            size_t r = (size_t)rr;
            if (r >= st && r < en) continue;
            size_t row = qlp_row(c, Ql, r);
            uint64_t p = c->moduli[row];
            uint64_t mat[64];
            for (size_t i = 0; i < sz; i++) mat[i] = punctured_mod(c->moduli + st, sz, i, p);
            uint64_t *dst = slab + r * N;
            for (size_t k = 0; k < N; k++) {
                u128 acc = 0;
                for (size_t i = 0; i < sz; i++) acc += (u128)t[(st + i) * N + k] * mat[i];
                dst[k] = (uint64_t)(acc % p);
            }
            fwd_limb(c, dst, row);
        }
    }
    free(t);
}

/* key_switch_inner_prod_c2_and_evk (src/eval_key_switch.cu:175-230):
 * cx[k][r] = sum_{b < beta} t_mod_up[b][r] * key[b][k][row(r)]  mod q_row(r),
 * accumulated in 128 bits and folded to its residue every 32 digits (with
 * primes below 2^61 a product is below 2^122, so 65 products of 61-bit
 * residues would pass 2^128), i.e. the exact sum mod q. */
void orc_ks_inner_prod(const orc_ctx *c, size_t chain_index, const uint64_t *t_mod_up, const uint64_t *key,
                       size_t key_dnum, uint64_t *cx) {
    (void)key_dnum;
    size_t N = c->N, alpha = c->size_P, Ql = size_Ql(c, chain_index), QlP = Ql + alpha, QP = c->size_QP;
    size_t beta = (Ql + alpha - 1) / alpha;
    for (size_t r = 0; r < QlP; r++) {
        size_t row = qlp_row(c, Ql, r);
        uint64_t q = c->moduli[row];
        for (size_t k = 0; k < N; k++) {
            u128 acc0 = 0, acc1 = 0;
            for (size_t b = 0; b < beta; b++) {
                uint64_t x = t_mod_up[(b * QlP + r) * N + k];
                acc0 += (u128)x * key[((b * 2 + 0) * QP + row) * N + k];
                acc1 += (u128)x * key[((b * 2 + 1) * QP + row) * N + k];
                if ((b & 31) == 31) {
                    acc0 %= q;
                    acc1 %= q;
                }
            }
            cx[r * N + k] = (uint64_t)(acc0 % q);
            cx[(QlP + r) * N + k] = (uint64_t)(acc1 % q);
        }
    }
}

/* moddown_from_NTT (src/rns_bconv.cu:776-828) for CKKS:
 *   INTT the P limbs; delta = fast BConv P -> Ql (bConv_BEHZ, :212-229;
 *   alpha == 1: moddown_bconv_single_p_kernel, :698-714);
 *   out_i = (cx_i - NTT(delta)_i) * P^-1 mod q_i  (FuseModDownEpilogue,
 *   include/ntt_radix8_tmpl.cuh:216-233). */
void orc_moddown(const orc_ctx *c, size_t chain_index, uint64_t *cx, uint64_t *out, int threads) {
    size_t N = c->N, alpha = c->size_P, Ql = size_Ql(c, chain_index);
    const uint64_t *P = c->moduli + c->size_Q;
    for (size_t j = 0; j < alpha; j++) {
        uint64_t p = P[j];
        inv_limb(c, cx + (Ql + j) * N, c->size_Q + j);
        uint64_t hinv = orc_invmod(punctured_mod(P, alpha, j, p), p), hs = orc_shoup(hinv, p);
        for (size_t k = 0; k < N; k++) cx[(Ql + j) * N + k] = mul_shoup(cx[(Ql + j) * N + k], hinv, hs, p);
    }
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
    for (long ii = 0; ii < (long)Ql; ii++) {
        size_t i = (size_t)ii;
        uint64_t q = c->moduli[i];
        uint64_t mat[64];
        for (size_t j = 0; j < alpha; j++) mat[j] = punctured_mod(P, alpha, j, q);
        uint64_t *d = (uint64_t *)malloc(N * sizeof(uint64_t));
        for (size_t k = 0; k < N; k++) {
            u128 acc = 0;
            for (size_t j = 0; j < alpha; j++) acc += (u128)cx[(Ql + j) * N + k] * mat[j];
            d[k] = (uint64_t)(acc % q);
        }
        fwd_limb(c, d, i);
        uint64_t pm = 1 % q;
        for (size_t j = 0; j < alpha; j++) pm = orc_mulmod(pm, P[j] % q, q);
        uint64_t pinv = orc_invmod(pm, q), ps = orc_shoup(pinv, q);
        for (size_t k = 0; k < N; k++) out[i * N + k] = mul_shoup(sub_mod(cx[i * N + k], d[k], q), pinv, ps, q);
        free(d);
    }
}

int orc_keyswitch(const orc_ctx *c, size_t chain_index, uint64_t *ct, const uint64_t *c2, const uint64_t *key,
                  size_t key_dnum, int threads) {
    size_t N = c->N, alpha = c->size_P, Ql = size_Ql(c, chain_index), QlP = Ql + alpha;
    size_t beta = (Ql + alpha - 1) / alpha;
    if (alpha == 0 || beta > key_dnum) return -1;
    uint64_t *tm = (uint64_t *)malloc(beta * QlP * N * sizeof(uint64_t));
    uint64_t *cx = (uint64_t *)malloc(2 * QlP * N * sizeof(uint64_t));
    uint64_t *o = (uint64_t *)malloc(Ql * N * sizeof(uint64_t));
    orc_modup(c, chain_index, c2, tm, threads);
    orc_ks_inner_prod(c, chain_index, tm, key, key_dnum, cx);
    for (size_t k = 0; k < 2; k++) {
        orc_moddown(c, chain_index, cx + k * QlP * N, o, threads);
        for (size_t i = 0; i < Ql; i++) {
            uint64_t q = c->moduli[i];
            uint64_t *dst = ct + (k * Ql + i) * N;
            for (size_t n = 0; n < N; n++) dst[n] = add_mod(dst[n], o[i * N + n], q);
        }
    }
    free(tm);
    free(cx);
    free(o);
    return 0;
}

int orc_multiply_and_relin(const orc_ctx *c, size_t chain_index, const uint64_t *a, const uint64_t *b,
                           const uint64_t *rlk, size_t key_dnum, uint64_t *out, int threads) {
    size_t N = c->N, Ql = size_Ql(c, chain_index);
    uint64_t *t3 = (uint64_t *)malloc(3 * Ql * N * sizeof(uint64_t));
    if (a == b)
        orc_tensor_square(c, Ql, a, t3);
    else
        orc_tensor(c, Ql, a, b, t3);
    int rc = orc_keyswitch(c, chain_index, t3, t3 + 2 * Ql * N, rlk, key_dnum, threads);
    memcpy(out, t3, 2 * Ql * N * sizeof(uint64_t));
    free(t3);
    return rc;
}

/* divide_and_round_q_last_ntt (src/rns.cu:1128-1184): floor division by q_last,
 *   out_j = (c_j - NTT_j([INTT_last(c_last)]_{q_j})) * q_last^-1  mod q_j. */
void orc_rescale(const orc_ctx *c, size_t chain_index, const uint64_t *in, size_t size, uint64_t *out,
                 int threads) {
    size_t N = c->N, L = size_Ql(c, chain_index);
    uint64_t ql = c->moduli[L - 1];
    uint64_t *last = (uint64_t *)malloc(N * sizeof(uint64_t));
    for (size_t s = 0; s < size; s++) {
        const uint64_t *ci = in + s * L * N;
        uint64_t *co = out + s * (L - 1) * N;
        memcpy(last, ci + (L - 1) * N, N * sizeof(uint64_t));
        inv_limb(c, last, L - 1);
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
        for (long jj = 0; jj < (long)(L - 1); jj++) {
            size_t j = (size_t)jj;
            uint64_t q = c->moduli[j];
            uint64_t *d = co + j * N;
            for (size_t k = 0; k < N; k++) d[k] = last[k] % q;
            fwd_limb(c, d, j);
            uint64_t inv = orc_invmod(ql % q, q), is = orc_shoup(inv, q);
            for (size_t k = 0; k < N; k++) d[k] = mul_shoup(sub_mod(ci[j * N + k], d[k], q), inv, is, q);
        }
    }
    free(last);
}

/* ------------------------------------------------------------------------ */
/* Galois                                                                    */
/* ------------------------------------------------------------------------ */

/* get_elt_from_step (include/galois.cuh:16-49) */
uint32_t orc_elt_from_step(int step, uint64_t N) {
    uint32_t n = (uint32_t)N, m32 = n * 2;
    uint64_t m = m32;
    if (step == 0) return (uint32_t)(m - 1);
    int sign = step < 0;
    uint32_t pos = (uint32_t)(step < 0 ? -step : step);
    if (pos >= (n >> 1)) return 0;
    pos &= m32 - 1;
    int s = sign ? (int)(n >> 1) - (int)pos : (int)pos;
    uint64_t g = 1;
    while (s--) g = (g * 5) & (m - 1);
    return (uint32_t)g;
}

/* permutation table (include/galois.cuh:98-113) */
void orc_galois_perm(uint64_t N, uint32_t elt, uint32_t *perm) {
    int logn = ilog2(N);
    for (uint64_t i = 0; i < N; i++) {
        uint32_t rev = brv((uint32_t)(N + i), logn + 1);
        uint64_t raw = ((uint64_t)elt * rev) >> 1;
        raw &= N - 1;
        perm[i] = brv((uint32_t)raw, logn);
    }
}

/* apply_galois_ntt_permutation (src/galois.cu:11-18): dst[i] = src[perm[i]] per limb */
void orc_apply_galois_ntt(uint64_t N, uint32_t elt, const uint64_t *src, uint64_t *dst, size_t L) {
    uint32_t *perm = (uint32_t *)malloc(N * sizeof(uint32_t));
    orc_galois_perm(N, elt, perm);
    for (size_t l = 0; l < L; l++)
        for (uint64_t i = 0; i < N; i++) dst[l * N + i] = src[l * N + perm[i]];
    free(perm);
}

int orc_apply_galois(const orc_ctx *c, size_t chain_index, uint64_t *ct, uint32_t elt, const uint64_t *key,
                     size_t key_dnum, int threads) {
    size_t N = c->N, Ql = size_Ql(c, chain_index);
    uint64_t *tmp = (uint64_t *)malloc(Ql * N * sizeof(uint64_t));
    orc_apply_galois_ntt(N, elt, ct, tmp, Ql);
    memcpy(ct, tmp, Ql * N * sizeof(uint64_t));
    orc_apply_galois_ntt(N, elt, ct + Ql * N, tmp, Ql);
    memset(ct + Ql * N, 0, Ql * N * sizeof(uint64_t));
    int rc = orc_keyswitch(c, chain_index, ct, tmp, key, key_dnum, threads);
    free(tmp);
    return rc;
}

int orc_hoist_rotations(const orc_ctx *c, size_t chain_index, const uint64_t *ct, const uint32_t *elts,
                        size_t n_elts, const uint64_t *const *keys, size_t key_dnum, uint64_t *out, int threads) {
    size_t N = c->N, alpha = c->size_P, Ql = size_Ql(c, chain_index), QlP = Ql + alpha;
    size_t beta = (Ql + alpha - 1) / alpha;
    if (alpha == 0 || beta > key_dnum) return -1;
    uint64_t *mu = (uint64_t *)malloc(beta * QlP * N * sizeof(uint64_t));
    uint64_t *mur = (uint64_t *)malloc(beta * QlP * N * sizeof(uint64_t));
    uint64_t *cx = (uint64_t *)malloc(2 * QlP * N * sizeof(uint64_t));
    uint64_t *o = (uint64_t *)malloc(Ql * N * sizeof(uint64_t));
    orc_modup(c, chain_index, ct + Ql * N, mu, threads);
    for (size_t e = 0; e < n_elts; e++) {
        uint64_t *dst = out + e * 2 * Ql * N;
        orc_apply_galois_ntt(N, elts[e], ct, dst, Ql);
        for (size_t b = 0; b < beta; b++)
            orc_apply_galois_ntt(N, elts[e], mu + b * QlP * N, mur + b * QlP * N, QlP);
        orc_ks_inner_prod(c, chain_index, mur, keys[e], key_dnum, cx);
        orc_moddown(c, chain_index, cx, o, threads);
        for (size_t i = 0; i < Ql; i++) {
            uint64_t q = c->moduli[i];
            for (size_t n = 0; n < N; n++) dst[i * N + n] = add_mod(dst[i * N + n], o[i * N + n], q);
        }
        orc_moddown(c, chain_index, cx + QlP * N, dst + Ql * N, threads);
    }
    free(mu);
    free(mur);
    free(cx);
    free(o);
    return 0;
}

/* hoisting_inplace (src/evaluate.cu:1732-1927): sum of the rotations by elts;
 * the inner products of all rotations are accumulated in the QlP basis and
 * moved down once:  out0 = sum sigma_e(c0) + ModDown(acc0), out1 = ModDown(acc1). */
int orc_hoisting(const orc_ctx *c, size_t chain_index, const uint64_t *ct, const uint32_t *elts, size_t n_elts,
                 const uint64_t *const *keys, size_t key_dnum, uint64_t *out, int threads) {
    size_t N = c->N, alpha = c->size_P, Ql = size_Ql(c, chain_index), QlP = Ql + alpha;
    size_t beta = (Ql + alpha - 1) / alpha;
    if (alpha == 0 || beta > key_dnum || n_elts == 0) return -1;
    uint64_t *mu = (uint64_t *)malloc(beta * QlP * N * sizeof(uint64_t));
    uint64_t *mur = (uint64_t *)malloc(beta * QlP * N * sizeof(uint64_t));
    uint64_t *cx = (uint64_t *)malloc(2 * QlP * N * sizeof(uint64_t));
    uint64_t *acc = (uint64_t *)calloc(2 * QlP * N, sizeof(uint64_t));
    uint64_t *c0 = (uint64_t *)calloc(Ql * N, sizeof(uint64_t));
    uint64_t *t0 = (uint64_t *)malloc(Ql * N * sizeof(uint64_t));
    orc_modup(c, chain_index, ct + Ql * N, mu, threads);
    for (size_t e = 0; e < n_elts; e++) {
        orc_apply_galois_ntt(N, elts[e], ct, t0, Ql);
        for (size_t i = 0; i < Ql; i++)
            for (size_t k = 0; k < N; k++) c0[i * N + k] = add_mod(c0[i * N + k], t0[i * N + k], c->moduli[i]);
        for (size_t b = 0; b < beta; b++)
            orc_apply_galois_ntt(N, elts[e], mu + b * QlP * N, mur + b * QlP * N, QlP);
        orc_ks_inner_prod(c, chain_index, mur, keys[e], key_dnum, cx);
        for (size_t h = 0; h < 2; h++)
            for (size_t r = 0; r < QlP; r++) {
                uint64_t q = c->moduli[qlp_row(c, Ql, r)];
                for (size_t k = 0; k < N; k++) {
                    size_t o = (h * QlP + r) * N + k;
                    acc[o] = add_mod(acc[o], cx[o], q);
                }
            }
    }
    orc_moddown(c, chain_index, acc, out, threads);
    for (size_t i = 0; i < Ql; i++)
        for (size_t k = 0; k < N; k++) out[i * N + k] = add_mod(out[i * N + k], c0[i * N + k], c->moduli[i]);
    orc_moddown(c, chain_index, acc + QlP * N, out + Ql * N, threads);
    free(mu);
    free(mur);
    free(cx);
    free(acc);
    free(c0);
    free(t0);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* key switching key (src/secretkey.cu:236-299, :354-398; polymath.cu:318-372) */
/* ------------------------------------------------------------------------ */

void orc_kswitch_key(const orc_ctx *c, const uint64_t *new_key, const uint64_t *s, const uint64_t *a,
                     const uint64_t *e_ntt, uint64_t *key_out) {
    size_t N = c->N, QP = c->size_QP, alpha = c->size_P, dnum = orc_dnum(c);
    const uint64_t *P = c->moduli + c->size_Q;
    for (size_t d = 0; d < dnum; d++) {
        uint64_t *b0 = key_out + (d * 2 + 0) * QP * N;
        uint64_t *b1 = key_out + (d * 2 + 1) * QP * N;
        for (size_t j = 0; j < QP; j++) {
            uint64_t q = c->moduli[j];
            uint64_t pm = 1 % q;
            for (size_t k = 0; k < alpha; k++) pm = orc_mulmod(pm, P[k] % q, q);
            int own = (j >= d * alpha && j < (d + 1) * alpha);
            for (size_t n = 0; n < N; n++) {
                size_t t = j * N + n;
                uint64_t av = a[d * QP * N + t];
                uint64_t red = (uint64_t)(((u128)av * s[t] + e_ntt[d * QP * N + t]) % q);
                uint64_t v = red ? q - red : 0;
                if (own) v = add_mod(v, orc_mulmod(pm, new_key[t], q), q);
                b0[t] = v;
                b1[t] = av;
            }
        }
    }
}
