/*
 * phantom_amd.h -- C ABI of the MI355X (gfx950) CKKS evaluation core.
 *
 * Drop-in boundary for the data-parallel hot path of gold9598/phantom-fhe:
 * batched negacyclic RNS NTT/INTT, ModUp/ModDown fast base conversion, the
 * hybrid key-switching inner product, the Galois automorphism and rescale.
 * Each entry point names the reference interface it replaces (file:line in
 * the reference tree).
 *
 * Conventions
 *   - All residue buffers are DEVICE pointers to uint64 residues, limb-major:
 *       limb = N residues of one prime, poly = [L][N], ciphertext = [size][L][N]
 *     (the reference's layout, include/ciphertext.h:7-308).
 *   - Keys are contiguous [dnum][2][|QP|][N] in NTT form, row 0 =
 *     -(a s + e) + [P]_q s' on digit d's own alpha limbs, row 1 = a
 *     (src/secretkey.cu:354-398).  The reference keeps the same rows behind an
 *     array of per-digit pointers.
 *   - chain_index follows the reference's context chain (src/context.cu:121-168):
 *     0 = key level (all |QP| primes), chain c >= 1 holds |Ql| = |Q| - c + 1
 *     data primes.
 *   - stream: a hipStream_t; NULL means hipStreamPerThread, the counterpart of
 *     the reference's cudaStreamPerThread (src/evaluate.cu:1079).  Calls are
 *     asynchronous on that stream.
 *   - Every function returns PFA_OK or an error code; pfa_last_error() gives
 *     the calling thread's message.  Codes map to the reference's exception
 *     classes: INVALID_ARGUMENT = std::invalid_argument (ValueError in
 *     Python), LOGIC = std::logic_error, RUNTIME = std::runtime_error
 *     (PHANTOM_CHECK_CUDA, include/cuda_wrapper.cuh:19-43).
 *   - Temporaries come from a device workspace kept per (host thread, stream)
 *     and grown on first use, where the reference makes stream-ordered
 *     allocations (cuda_auto_ptr, include/cuda_wrapper.cuh:185-189); calls in
 *     steady state allocate nothing.  The first key switch of a (level,
 *     batch) shape also builds and uploads its base-conversion work schedule
 *     (kept with the context), so a shape's first call must not be captured.
 */
#ifndef PHANTOM_AMD_H
#define PHANTOM_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PFA_OK 0
#define PFA_ERR_INVALID_ARGUMENT 1
#define PFA_ERR_LOGIC 2
#define PFA_ERR_RUNTIME 3

typedef struct pfa_context pfa_context;

/* Message of the last failed call on this thread ("" if none). */
const char *pfa_last_error(void);

/* ABI version of this library. */
int pfa_abi_version(void);

/* ------------------------------------------------------------------ setup */

/* CoeffModulus::Create (src/host/modulus.cu:80-111; python binding
 * create_coeff_modulus, python/src/binding.cu:56).  out[count]. */
int pfa_create_coeff_modulus(uint64_t poly_degree, const int *bit_sizes, size_t count, uint64_t *out);

/* PhantomContext::PhantomContext (src/context.cu:121-183): builds the chain,
 * the NTT tables of all |QP| primes (minimal primitive 2N-th root, bit-reversed
 * powers, N^-1 folded, src/host/ntt.cu:11-56) and the per-level RNS constants
 * (src/rns.cu:11-195) on `device`.  moduli = the |Q| data primes followed by
 * the special_size special primes, as EncryptionParameters::coeff_modulus. */
int pfa_context_create(uint64_t poly_degree, const uint64_t *moduli, size_t size_QP, size_t special_size,
                       int device, pfa_context **out);
void pfa_context_destroy(pfa_context *ctx);

/* Copies the minimal primitive 2N-th root of every prime (|QP| values). */
int pfa_context_roots(const pfa_context *ctx, uint64_t *out);

/* cudaStreamSynchronize under PHANTOM_CHECK_CUDA (include/cuda_wrapper.cuh:19-43),
 * plus the errors kernels of this context recorded on the device: waits for
 * `stream`, then returns PFA_ERR_RUNTIME if a kernel recorded one of
 *   - a single-launch NTT (opt-in with PFA_NTT_FLOW=1, batches of 8+ limbs at
 *     N = 2^16) whose bounded wait expired or that did not transform every tile;
 *   - a key-switch inner product (every key switch: relinearize,
 *     multiply_and_relin, rotations, hoisting, BSGS, bootstrapping) whose split
 *     item's digit chunks did not all run on one XCD.  Items are split only on
 *     a device that deals workgroups to its XCDs round-robin (probed when the
 *     context is created), so this is a consistency check of that probe.
 * Every later call that takes this context (any entry point with a `ctx`
 * argument) also returns such a record, before it launches anything, once the
 * kernel that recorded it has run; the record is cleared once returned.  So
 * after key switches or single-launch NTTs, call this before trusting their
 * outputs.  The reference's kernels record no errors. */
int pfa_synchronize(const pfa_context *ctx, void *stream);

/* ------------------------------------------------------------------ NTT */

/* nwt_2d_radix8_forward_inplace[_batched] (include/ntt.cuh:173, :184;
 * src/ntt/fntt_2d.cu:665-784): in-place forward NTT of M polys x L limbs,
 * limb l of each poly using table row start + l. */
int pfa_ntt_forward(const pfa_context *ctx, uint64_t *inout, size_t M, size_t L, size_t start, void *stream);

/* nwt_2d_radix8_backward_inplace (include/ntt.cuh:216; src/ntt/intt_2d.cu:769-813),
 * batched over M polys like the forward. */
int pfa_ntt_inverse(const pfa_context *ctx, uint64_t *inout, size_t M, size_t L, size_t start, void *stream);

/* No reference counterpart (a query for tests and tools): *out = 1 if an NTT of
 * M polys x L limbs on this context runs as the single launch whose
 * intermediate stays in one XCD's L2 (opted into with PFA_NTT_FLOW=1 at context
 * creation, N = 2^16, M L >= 8, the device deals workgroups to 8 XCDs
 * round-robin), 0 if it runs as two launches. */
int pfa_ntt_single_launch(const pfa_context *ctx, size_t M, size_t L, int *out);

/* No reference counterpart (a measurement aid): copies n uint64 words (n even,
 * dst and src 16-byte aligned) from src to dst with nontemporal 16-byte loads
 * and stores, on `workgroups`
 * workgroups of 256 threads (0: one per 16 KiB), the achievable one-read
 * one-write bandwidth against which the NTT is measured. */
int pfa_stream_copy(uint64_t *dst, const uint64_t *src, size_t n, size_t workgroups, void *stream);

/* --------------------------------------------------- RNS / key switching */

/* DRNSTool::modup (include/rns.cuh:156; src/rns_bconv.cu:530-628):
 * c2 [|Ql|][N] (NTT form) -> t_mod_up [beta][|Ql|+alpha][N]. */
int pfa_modup(const pfa_context *ctx, size_t chain_index, const uint64_t *c2, uint64_t *t_mod_up, void *stream);

/* key_switch_inner_prod (include/evaluate.cuh:41-43; kernel
 * src/eval_key_switch.cu:175-230): cx [2][|Ql|+alpha][N]. */
int pfa_ks_inner_prod(const pfa_context *ctx, size_t chain_index, const uint64_t *t_mod_up, const uint64_t *key,
                      size_t key_dnum, uint64_t *cx, void *stream);

/* DRNSTool::moddown_from_NTT (include/rns.cuh; src/rns_bconv.cu:776-828):
 * cx_k [|Ql|+alpha][N] -> out [|Ql|][N] = (cx - NTT(BConv_P->Ql(INTT(cx_P)))) * P^-1.
 * cx_k is not modified. */
int pfa_moddown(const pfa_context *ctx, size_t chain_index, const uint64_t *cx_k, uint64_t *out, void *stream);

/* keyswitch_inplace (include/evaluate.cuh:45-48; src/eval_key_switch.cu:294-381):
 * ct[0..1] ([2][|Ql|][N]) += ModDown(<ModUp(c2), key>). */
int pfa_keyswitch(const pfa_context *ctx, size_t chain_index, uint64_t *ct, const uint64_t *c2, const uint64_t *key,
                  size_t key_dnum, void *stream);

/* ------------------------------------------------------------ evaluator */

/* bgv_ckks_multiply's tensor (src/evaluate.cu:345-397 -> tensor_prod_2x2_rns_poly,
 * src/polymath.cu:463-498): a, b [2][|Ql|][N] -> out [3][|Ql|][N].  a, b and
 * out must be 16-byte aligned (the kernel moves residue pairs); a misaligned
 * pointer returns PFA_ERR_INVALID_ARGUMENT.  The same holds for a, b and out of
 * pfa_multiply_and_relin, pfa_multiply_relin_rescale and their _batch forms. */
int pfa_tensor(const pfa_context *ctx, size_t chain_index, const uint64_t *a, const uint64_t *b, uint64_t *out,
               void *stream);

/* multiply_and_relin_inplace (src/evaluate.cu:1061-1104): out [2][|Ql|][N].
 * a, b, out 16-byte aligned (as pfa_tensor). */
int pfa_multiply_and_relin(const pfa_context *ctx, size_t chain_index, const uint64_t *a, const uint64_t *b,
                           const uint64_t *rlk, size_t key_dnum, uint64_t *out, void *stream);

/* relinearize_inplace (src/evaluate.cu:1342-1374): ct3 [3][|Ql|][N] -> out [2][|Ql|][N]. */
int pfa_relinearize(const pfa_context *ctx, size_t chain_index, const uint64_t *ct3, const uint64_t *rlk,
                    size_t key_dnum, uint64_t *out, void *stream);

/* rescale_to_next -> divide_and_round_q_last_ntt (src/evaluate.cu:1582-1602,
 * src/rns.cu:1128-1184): in [size][|Ql|][N] -> out [size][|Ql|-1][N] (floor). */
int pfa_rescale(const pfa_context *ctx, size_t chain_index, const uint64_t *in, size_t size, uint64_t *out,
                void *stream);

/* No counterpart in the reference: pfa_rescale for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops or
 * harnesses that forbid hipMalloc).  Same residues as pfa_rescale; allocates
 * nothing: the base conversion's intermediate is formed in `out`, and the last
 * limb's coefficients go to a static per-device scratch array of 4 MiB
 * (size x N <= 524288 residues: 8 polys at N = 2^16; larger calls return
 * PFA_ERR_INVALID_ARGUMENT).  `in` and `out` must not overlap.  Calls that
 * overlap in time on one device share that scratch and race; calls on one
 * stream are ordered.  The single-launch NTT is never used here. */
int pfa_rescale_noalloc(const pfa_context *ctx, size_t chain_index, const uint64_t *in, size_t size, uint64_t *out,
                        void *stream);

/* multiply_and_relin_inplace then rescale_to_next_inplace (src/evaluate.cu:1061-1104,
 * :1582-1602) as one call: out [2][|Ql|-1][N] = rescale(multiply_and_relin(a, b)),
 * bit-identical to pfa_multiply_and_relin followed by pfa_rescale.  The ModDown
 * output is never formed: its last limb's coefficients come from the ModDown
 * inputs and the two forward NTTs of the rescale and the ModDown merge by
 * linearity.  out must not alias a or b; |Ql| >= 2. */
int pfa_multiply_relin_rescale(const pfa_context *ctx, size_t chain_index, const uint64_t *a, const uint64_t *b,
                               const uint64_t *rlk, size_t key_dnum, uint64_t *out, void *stream);

/* multiply_and_relin_inplace (src/evaluate.cu:1061-1104) over `count`
 * independent pairs with one relinearization key, in one set of launches:
 * a, b, out [count][2][|Ql|][N]; member i's residues equal pfa_multiply_and_relin
 * of a[i], b[i].  out may equal a or b but not overlap them otherwise. */
int pfa_multiply_and_relin_batch(const pfa_context *ctx, size_t chain_index, size_t count, const uint64_t *a,
                                 const uint64_t *b, const uint64_t *rlk, size_t key_dnum, uint64_t *out,
                                 void *stream);

/* pfa_multiply_relin_rescale (multiply_and_relin_inplace then
 * rescale_to_next_inplace, src/evaluate.cu:1061-1104, :1582-1602) over `count`
 * independent pairs with one key: a, b [count][2][|Ql|][N] -> out
 * [count][2][|Ql|-1][N], member i equal to pfa_multiply_relin_rescale of a[i],
 * b[i].  out must not overlap a or b; |Ql| >= 2. */
int pfa_multiply_relin_rescale_batch(const pfa_context *ctx, size_t chain_index, size_t count, const uint64_t *a,
                                     const uint64_t *b, const uint64_t *rlk, size_t key_dnum, uint64_t *out,
                                     void *stream);

/* relinearize_inplace then rescale_to_next_inplace (src/evaluate.cu:1342-1374,
 * :1582-1602) as one call: ct3 [3][|Ql|][N] -> out [2][|Ql|-1][N], bit-identical to
 * pfa_relinearize followed by pfa_rescale.  out must not alias ct3. */
int pfa_relinearize_rescale(const pfa_context *ctx, size_t chain_index, const uint64_t *ct3, const uint64_t *rlk,
                            size_t key_dnum, uint64_t *out, void *stream);

/* get_elt_from_step (include/galois.cuh:16-49): 5^step mod 2N, step 0 -> 2N-1. */
int pfa_galois_elt_from_step(int step, uint64_t poly_degree, uint32_t *elt);

/* PhantomGaloisTool::apply_galois_ntt (include/galois.cuh:157; src/galois.cu:11-18,
 * :86-102): dst[l][i] = src[l][pi(i)] for L limbs; src != dst. */
int pfa_apply_galois_ntt(const pfa_context *ctx, uint32_t elt, const uint64_t *src, uint64_t *dst, size_t L,
                         void *stream);

/* apply_galois_with_ksk (src/evaluate.cu:1607-1656) on a size-2 ciphertext, in place. */
int pfa_apply_galois(const pfa_context *ctx, size_t chain_index, uint64_t *ct, uint32_t elt, const uint64_t *key,
                     size_t key_dnum, void *stream);

/* hoist_rotations (src/evaluate.cu:1929-2082): one ModUp of c1 shared by n
 * rotations; keys = host array of n device key pointers; out [n][2][|Ql|][N]. */
int pfa_hoist_rotations(const pfa_context *ctx, size_t chain_index, const uint64_t *ct, const uint32_t *elts,
                        size_t n, const uint64_t *const *keys, size_t key_dnum, uint64_t *out, void *stream);

/* hoisting_inplace (src/evaluate.cu:1732-1927): the sum of the n rotations
 * of ct, sharing one ModUp of c1; the inner products of all rotations are
 * accumulated before one ModDown.  out [2][|Ql|][N]. */
int pfa_hoisting(const pfa_context *ctx, size_t chain_index, const uint64_t *ct, const uint32_t *elts, size_t n,
                 const uint64_t *const *keys, size_t key_dnum, uint64_t *out, void *stream);

/* -------------------------------------------- key material and elementwise */

/* generate_one_kswitch_key (src/secretkey.cu:354-398, with
 * multiply_temp_mod_and_add_rns_poly, src/polymath.cu:318-336): all NTT form,
 * new_key, s [|QP|][N]; a, e [dnum][|QP|][N] -> key [dnum][2][|QP|][N]. */
int pfa_kswitch_key(const pfa_context *ctx, const uint64_t *new_key, const uint64_t *s, const uint64_t *a,
                    const uint64_t *e, uint64_t *key, void *stream);

/* Elementwise ops over L limbs using primes start..start+L-1
 * (add_rns_poly / sub_rns_poly / multiply_rns_poly / negate_rns_poly,
 * src/polymath.cu).  out may alias an input. */
int pfa_poly_add(const pfa_context *ctx, const uint64_t *a, const uint64_t *b, uint64_t *out, size_t L, size_t start,
                 void *stream);
int pfa_poly_sub(const pfa_context *ctx, const uint64_t *a, const uint64_t *b, uint64_t *out, size_t L, size_t start,
                 void *stream);
int pfa_poly_mul(const pfa_context *ctx, const uint64_t *a, const uint64_t *b, uint64_t *out, size_t L, size_t start,
                 void *stream);

/* multiply_plain_ntt (src/evaluate.cu:1224-1250): out[k] = ct[k] * pt over
 * limbs 0..L-1 for every poly k < size of ct [size][L][N] (NTT form), in one
 * launch (the reference launches one multiply per poly).  out may equal ct. */
int pfa_ct_multiply_plain(const pfa_context *ctx, const uint64_t *ct, size_t size, const uint64_t *pt, uint64_t *out,
                          size_t L, void *stream);
int pfa_poly_negate(const pfa_context *ctx, const uint64_t *a, uint64_t *out, size_t L, size_t start, void *stream);

/* Reduces signed 64-bit coefficients (one poly, N values) into L limbs using
 * primes start..start+L-1: out[l][i] = in[i] mod q_(start+l) (sampler output
 * decomposition, src/prng.cu / src/secretkey.cu:236-299). */
int pfa_poly_from_signed(const pfa_context *ctx, const int64_t *in, uint64_t *out, size_t L, size_t start,
                         void *stream);

/* ------------------------------------------------------------ CKKS encoder */

/* PhantomCKKSEncoder::encode (src/ckks.cu:71-137; special FFT src/fft.cu):
 * n_values <= N/2 complex slot values (device, interleaved re/im doubles;
 * missing slots are zero) times `scale`, rounded, into a plaintext of L limbs
 * (primes 0..L-1) in NTT form; a rounded coefficient of any size is reduced
 * into each prime exactly.  INVALID_ARGUMENT, as the reference, if
 * floor(log2(scale)) + 1 or ceil(log2(max |coefficient|)) + 1 reaches the
 * bit length of q_0 ... q_(L-1) ("scale out of bounds", "encoded values are
 * too large").  Synchronizes the stream. */
int pfa_ckks_encode(const pfa_context *ctx, const double *values, size_t n_values, double scale, uint64_t *out,
                    size_t L, void *stream);

/* PhantomCKKSEncoder::decode (src/ckks.cu:139-190): plaintext of L limbs in
 * NTT form -> N/2 complex slot values (device, interleaved re/im) divided by
 * `scale`.  Coefficients are composed from all L limbs and centred, exact for
 * any |m| < Q / 2 (compose_array, src/rns_base.cu:173-253).  INVALID_ARGUMENT
 * if floor(log2(scale)) reaches the bit length of q_0 ... q_(L-1). */
int pfa_ckks_decode(const pfa_context *ctx, const uint64_t *in, size_t L, double scale, double *values,
                    void *stream);

/* encode_single_chain_plaintext (src/single_chain_plaintext.cu:93-150): the
 * same slot encoding as pfa_ckks_encode (at chain index 1, with its bounds),
 * returned as the N rounded coefficients reduced mod q_0 and centred (device
 * int64) instead of residues -- the reference's level-independent plaintext.
 * Expand with pfa_expand_signed and pfa_ntt_forward at the level of use.
 * Synchronizes the stream. */
int pfa_ckks_encode_coeffs(const pfa_context *ctx, const double *values, size_t n_values, double scale,
                           int64_t *coeffs, void *stream);

/* ------------------------------------------------------------------ BSGS */

/* light_pt_expand_per_tower_kernel (src/bootstrap.cu, used by src/bsgs.cu:260-271)
 * batched: n signed coefficient polys in[n][N] -> out[n][L][N], the residues of
 * table rows start .. start+L-1 (coefficient form; NTT them with
 * pfa_ntt_forward(ctx, out, n, L, start, stream)). */
int pfa_expand_signed(const pfa_context *ctx, const int64_t *in, size_t n, uint64_t *out, size_t L, size_t start,
                      void *stream);

/* mac_accumulate_kernel (src/bsgs.cu:51-96) for every giant at once, the
 * accumulation of bsgs_apply_giants_with_babies (build_partial,
 * src/bsgs.cu:276-342):
 *   out[g][k] = sum_{b < M} pts[g*M + b] * babies[b][k]   (k = 0, 1; mod q_j)
 * pts: G*M plaintexts [Ql][N]; babies: M ciphertexts [2][Ql][N]; out: G
 * ciphertexts [2][Ql][N]; all NTT form at chain_index.  The pointer tables are
 * host arrays of device pointers. */
int pfa_bsgs_mac(const pfa_context *ctx, size_t chain_index, const uint64_t *const *pts,
                 const uint64_t *const *babies, size_t M, size_t G, uint64_t *const *out, void *stream);

/* The tiled layout of a BSGS plaintext set (D plaintexts of Ql <= 64 limbs at
 * one chain index, NTT form): one region per limb, in limb order; in limb j's
 * region, residues [512 t, 512 t + 512) of plaintext d sit at position
 * (t D + d) 512.  A limb whose prime is 2^40 or more stores 8 bytes per
 * residue; a limb whose prime is below 2^40 stores D N 32-bit low words
 * followed by D N bytes of bits 32..39 (5 bytes per residue).  It stores the
 * plaintexts the accumulation reads together next to each other, as few bytes
 * as the residues need.  Copies src [n][Ql][N] into positions d0 .. d0+n-1 of
 * a buffer of at least pfa_bsgs_tiled_size bytes.  Layout of this library (the
 * reference re-expands each plaintext per use, src/bsgs.cu:276-312). */
int pfa_bsgs_tile_plaintexts(const pfa_context *ctx, size_t chain_index, const uint64_t *src, size_t n,
                             uint64_t *tiled, size_t d0, size_t D, void *stream);

/* Bytes of a tiled set of D plaintexts at chain_index (see pfa_bsgs_tile_plaintexts). */
int pfa_bsgs_tiled_size(const pfa_context *ctx, size_t chain_index, size_t D, size_t *bytes);

/* pfa_bsgs_mac with the G*M plaintexts given as one tiled set (D = M*G,
 * plaintext g*M + b for giant g and baby b). */
int pfa_bsgs_mac_tiled(const pfa_context *ctx, size_t chain_index, const uint64_t *tiled,
                       const uint64_t *const *babies, size_t M, size_t G, uint64_t *const *out, void *stream);

/* apply_galois_with_ksk (src/evaluate.cu:1607-1656) over `count` ciphertexts,
 * each with its own Galois element and key, in one set of launches: in, out
 * [count][2][Ql][N] at chain_index, out[i] = rotate(in[i], elts[i]) with keys[i]
 * ([key_dnum][2][QP][N]); the same residues as count pfa_apply_galois calls.
 * out must not overlap in. */
int pfa_rotate_batch(const pfa_context *ctx, size_t chain_index, size_t count, const uint64_t *in,
                     const uint32_t *elts, const uint64_t *const *keys, size_t key_dnum, uint64_t *out,
                     void *stream);

/* compute_bsgs_babies (src/bsgs.cu:194-214): babies[0] = ct and
 * babies[b] = rotate(babies[b - msb(b)], msb(b)) for 1 <= b < M, each rotation
 * apply_galois_with_ksk (src/evaluate.cu:1607-1656) with the direct key.
 * ct [2][Ql][N] at chain_index; keys[k] is the Galois key of rotation step 2^k
 * ([key_dnum][2][QP][N]) for every 2^k < M; out receives all M babies as
 * [M][2][Ql][N] (out[0] a copy of ct; ct may be out itself).  The babies with
 * msb(b) = 2^k are independent, so each such level runs as one batched
 * rotation. */
int pfa_bsgs_babies(const pfa_context *ctx, size_t chain_index, const uint64_t *ct, size_t M,
                    const uint64_t *const *keys, size_t key_dnum, uint64_t *out, void *stream);

/* The giant-step stage of bsgs_apply_giants_with_babies (src/bsgs.cu:344-356):
 * acc = partial[G-1]; acc = rotate(acc, step) + partial[g] for g = G-2 .. 0;
 * out = rescale_to_next(acc).  partials [G][2][Ql][N] (NTT form, chain_index)
 * are overwritten: partial[g] ends holding the accumulator at g.  key is the
 * Galois key of `step` (unused when G = 1); out is [2][Ql-1][N]. */
int pfa_bsgs_giants(const pfa_context *ctx, size_t chain_index, uint64_t *partials, size_t G, int step,
                    const uint64_t *key, size_t key_dnum, uint64_t *out, void *stream);

/* bsgs_apply_giants_with_babies (src/bsgs.cu:216-357) over a tiled plaintext
 * set (D = M*G, see pfa_bsgs_tile_plaintexts): the accumulation of every
 * giant's partial (pfa_bsgs_mac_tiled), the Horner loop with rotation step M
 * and the rescale (pfa_bsgs_giants), in one call.  babies: M ciphertexts
 * [2][Ql][N]; key: the Galois key of step M (unused when G = 1); out
 * [2][Ql-1][N].  Temporaries: G ciphertexts of workspace. */
int pfa_bsgs_apply_giants(const pfa_context *ctx, size_t chain_index, const uint64_t *tiled,
                          const uint64_t *const *babies, size_t M, size_t G, const uint64_t *key, size_t key_dnum,
                          uint64_t *out, void *stream);

/* ------------------------------------------------------------ bootstrapping */

/* The raise step of mod_raise_inplace (mod_raise_extend_modulus and
 * mod_raise_signed_tile_kernel, src/bootstrap.cu:37-75, :105-180): `in` holds
 * `size` polys [size][1][N] at the bottom of the chain (the single prime q0,
 * table row 0, NTT form); out [size][|Q|][N] receives, over every prime of the
 * first data level (chain index 1), each coefficient read as the centred
 * integer (v - q0 when v >= floor(q0 / 2)), in NTT form.  Temporaries:
 * size x N words of workspace. */
int pfa_mod_raise(const pfa_context *ctx, const uint64_t *in, size_t size, uint64_t *out, void *stream);

/* Linear combination of ciphertexts with integer constants, the weighted sum
 * of Chebyshev terms before its one rescale (weighted_sum_chebyshev,
 * src/evalmod.cu:277-335):
 *   out[k][l] = sum_t consts[t] ins[t][k][l]  (+ bias on poly 0 of each ciphertext)  mod q_l
 * for polys k < size and limbs l < L (table rows 0 .. L-1), NTT form; the
 * size polys are size / ct_size ciphertexts of ct_size polys each (ct_size =
 * size for one ciphertext), and the bias goes to polys k with k mod ct_size = 0.
 * ins[t] is [size][in_limbs[t]][N] with in_limbs[t] >= L: a ciphertext at a
 * lower chain index enters as it is (its first L limbs are read).  consts are
 * signed; bias points to a signed 128-bit integer as two words (low, high;
 * two's complement) or is NULL.  n <= 8.  out may be one of the inputs when
 * that input has exactly L limbs. */
int pfa_ct_lincomb(const pfa_context *ctx, size_t L, size_t size, size_t ct_size, const uint64_t *const *ins,
                   const size_t *in_limbs, const int64_t *consts, size_t n, const uint64_t *bias, uint64_t *out,
                   void *stream);

#ifdef __cplusplus
}
#endif
#endif /* PHANTOM_AMD_H */
