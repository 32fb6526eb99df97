/*
 * CPU oracle for the CKKS evaluation hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker that the HIP
 * product path is compared against, and the "port" CPU baseline that
 * bench.py times.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.  The product (phantom-fhe_amd/) never links,
 * imports or calls it.
 *
 * Every function restates the arithmetic of the reference
 * (gold9598/phantom-fhe) from the mathematics, citing the reference
 * file:line it follows.  All residues are canonical, i.e. in [0, q).
 *
 * Layouts (identical to the reference and to the product):
 *   limb       = N uint64 residues of one RNS prime
 *   poly       = [L][N] limbs, limb-major
 *   ciphertext = [size][L][N]
 *   key        = [dnum][2][|QP|][N]   (row 0 = -(a s + e) + [P]_q s' on the
 *                digit's own alpha limbs, row 1 = a), NTT form
 *
 * Parity pinning: see tests/test_oracle_*.py.  Each function is checked there
 * against an independent restatement (Python big integers / brute force) or a
 * closed-form identity.
 */
#ifndef CKKS_ORACLE_H
#define CKKS_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- number theory (src/host/numth.cu, src/host/modulus.cu) ---- */
int orc_is_prime(uint64_t n);
/* CoeffModulus::Create: returns 0 on success, -1 when not enough primes. */
int orc_create_coeff_modulus(uint64_t N, const int *bit_sizes, size_t count, uint64_t *out);
uint64_t orc_minimal_primitive_root(uint64_t degree, uint64_t q);
uint64_t orc_mulmod(uint64_t a, uint64_t b, uint64_t q);
uint64_t orc_powmod(uint64_t a, uint64_t e, uint64_t q);
uint64_t orc_invmod(uint64_t a, uint64_t q);
uint64_t orc_shoup(uint64_t w, uint64_t q);

/* ---- NTT tables (src/host/ntt.cu:11-56) ---- */
void orc_ntt_tables(uint64_t N, uint64_t q, uint64_t *tw, uint64_t *tw_shoup,
                    uint64_t *itw, uint64_t *itw_shoup, uint64_t *ninv, uint64_t *ninv_shoup);

/* ---- single-limb transforms ---- */
void orc_ntt_fwd_limb(uint64_t *a, uint64_t N, uint64_t q, const uint64_t *tw, const uint64_t *tws);
void orc_ntt_inv_limb(uint64_t *a, uint64_t N, uint64_t q, const uint64_t *itw, const uint64_t *itws,
                      uint64_t ninv);
/* O(N^2) closed form: out[i] = sum_j a_j psi^((2 brv(i)+1) j) */
void orc_ntt_naive_limb(const uint64_t *a, uint64_t *out, uint64_t N, uint64_t q, uint64_t psi);

/* ---- context: key-level chain with all |QP| primes ---- */
typedef struct orc_ctx orc_ctx;
orc_ctx *orc_ctx_create(uint64_t N, const uint64_t *moduli, size_t size_QP, size_t size_P);
void orc_ctx_destroy(orc_ctx *ctx);
size_t orc_ctx_size_QP(const orc_ctx *ctx);
const char *orc_build_info(void);
const uint64_t *orc_ctx_table(const orc_ctx *ctx, size_t prime_idx, int which);
uint64_t orc_ctx_root(const orc_ctx *ctx, size_t prime_idx);

/* Batched NTT over M polys x L limbs using table rows start..start+L-1
 * (nwt_2d_radix8_forward_inplace[_batched], src/ntt/fntt_2d.cu:665-784). */
void orc_ntt_fwd(const orc_ctx *ctx, uint64_t *data, size_t M, size_t L, size_t start, int threads);
void orc_ntt_inv(const orc_ctx *ctx, uint64_t *data, size_t M, size_t L, size_t start, int threads);

/* (d0,d1,d2) = tensor of two size-2 ciphertexts at L limbs (src/polymath.cu:463-498) */
void orc_tensor(const orc_ctx *ctx, size_t L, const uint64_t *a, const uint64_t *b, uint64_t *out);
/* square variant (src/polymath.cu:500-532) */
void orc_tensor_square(const orc_ctx *ctx, size_t L, const uint64_t *a, uint64_t *out);

/* beta = ceil(|Ql| / alpha) at chain_index (src/rns.cu:152) */
size_t orc_beta(const orc_ctx *ctx, size_t chain_index);
/* ModUp (src/rns_bconv.cu:530-628): c2 [|Ql|][N] NTT form -> t_mod_up [beta][|QlP|][N] */
void orc_modup(const orc_ctx *ctx, size_t chain_index, const uint64_t *c2, uint64_t *t_mod_up, int threads);
/* Inner product (src/eval_key_switch.cu:175-230): cx [2][|QlP|][N] */
void orc_ks_inner_prod(const orc_ctx *ctx, size_t chain_index, const uint64_t *t_mod_up,
                       const uint64_t *key, size_t key_dnum, uint64_t *cx);
/* ModDown (src/rns_bconv.cu:776-828): cx_k [|QlP|][N] (P limbs are overwritten)
 * -> out [|Ql|][N] = (cx - NTT(delta)) * P^-1 */
void orc_moddown(const orc_ctx *ctx, size_t chain_index, uint64_t *cx_k, uint64_t *out, int threads);
/* keyswitch_inplace (src/eval_key_switch.cu:294-381): ct[0..1] += ModDown(<ModUp(c2), key>) */
int orc_keyswitch(const orc_ctx *ctx, size_t chain_index, uint64_t *ct, const uint64_t *c2,
                  const uint64_t *key, size_t key_dnum, int threads);
/* multiply_and_relin (src/evaluate.cu:1061-1104): out [2][|Ql|][N] */
int orc_multiply_and_relin(const orc_ctx *ctx, size_t chain_index, const uint64_t *a, const uint64_t *b,
                           const uint64_t *rlk, size_t key_dnum, uint64_t *out, int threads);
/* rescale (divide_and_round_q_last_ntt, src/rns.cu:1160-1184): in [size][L][N] -> out [size][L-1][N] */
void orc_rescale(const orc_ctx *ctx, size_t chain_index, const uint64_t *in, size_t size, uint64_t *out,
                 int threads);

/* ---- Galois (include/galois.cuh:16-131, src/galois.cu:11-18) ---- */
uint32_t orc_elt_from_step(int step, uint64_t N);
void orc_galois_perm(uint64_t N, uint32_t elt, uint32_t *perm);
void orc_apply_galois_ntt(uint64_t N, uint32_t elt, const uint64_t *src, uint64_t *dst, size_t L);
/* apply_galois_with_ksk (src/evaluate.cu:1607-1656) on a size-2 ciphertext, in place */
int orc_apply_galois(const orc_ctx *ctx, size_t chain_index, uint64_t *ct, uint32_t elt,
                     const uint64_t *key, size_t key_dnum, int threads);
/* hoist_rotations (src/evaluate.cu:1929-2082): out [n_elts][2][|Ql|][N] */
int orc_hoist_rotations(const orc_ctx *ctx, size_t chain_index, const uint64_t *ct, const uint32_t *elts,
                        size_t n_elts, const uint64_t *const *keys, size_t key_dnum, uint64_t *out, int threads);

/* hoisting_inplace (src/evaluate.cu:1732-1927): out [2][|Ql|][N] = sum of rotations */
int orc_hoisting(const orc_ctx *ctx, size_t chain_index, const uint64_t *ct, const uint32_t *elts, size_t n_elts,
                 const uint64_t *const *keys, size_t key_dnum, uint64_t *out, int threads);

/* ---- key construction (src/secretkey.cu:354-398, src/polymath.cu:318-372) ----
 * new_key, s: [|QP|][N] NTT form; a, e_ntt: [dnum][|QP|][N]; key_out: [dnum][2][|QP|][N] */
void orc_kswitch_key(const orc_ctx *ctx, const uint64_t *new_key, const uint64_t *s, const uint64_t *a,
                     const uint64_t *e_ntt, uint64_t *key_out);
size_t orc_dnum(const orc_ctx *ctx);

/* ---- elementwise helpers used by tests ---- */
void orc_mul_poly(const orc_ctx *ctx, size_t L, size_t start, const uint64_t *a, const uint64_t *b, uint64_t *out);

#ifdef __cplusplus
}
#endif
#endif
