// RNS / key-switching / evaluator kernels and their C-ABI entry points:
// ModUp, the key-switch inner product, ModDown, key switching, tensor,
// relinearization, rescale, the Galois automorphism, hoisted rotations, key
// construction and the elementwise poly ops.
//
// Every kernel emits canonical residues; each formula is the reference's
// (file:line given per kernel), so outputs are bit-identical to it.
#include <algorithm>

#include "internal.h"
#include "modarith.h"

namespace pfa {

namespace {

constexpr int kThreads = 256;
constexpr uint32_t kMaxAlpha = 16;  // special primes per digit supported by the BConv kernels

__device__ __forceinline__ uint64_t mulmod_b(uint64_t a, uint64_t b, uint64_t q, ulonglong2 r) {
    U128 p{a * b, mulhi64(a, b)};
    return barrett128(p, q, r.x, r.y);
}

// ------------------------------------------------------------ elementwise
enum BinOp { kAdd, kSub, kMul, kNeg };

__global__ void __launch_bounds__(kThreads)
k_poly_binop(int op, const uint64_t *a, const uint64_t *b, uint64_t *out, const uint64_t *mod,
             const ulonglong2 *ratio, uint32_t start, uint32_t N, uint64_t a_stride, uint64_t b_stride,
             uint64_t out_stride) {
    // poly blockIdx.z of a batch: a, b, out advanced by their strides (b_stride
    // 0: one b for every poly)
    const uint32_t l = blockIdx.y, n = blockIdx.x * kThreads + threadIdx.x, k = blockIdx.z;
    a += k * a_stride;
    b += k * b_stride;
    out += k * out_stride;
    const uint64_t q = mod[start + l];
    const size_t i = (size_t)l * N + n;
    const uint64_t x = a[i];
    uint64_t r;
    switch (op) {
    case kAdd: r = add_mod(x, b[i], q); break;
    case kSub: r = sub_mod(x, b[i], q); break;
    case kMul:
        if (q < kF64PrimeBound) {
            const ArithF64 ar(q);
            const double y = ar.load(b[i]);
            r = ar.store(ar.mulw(ar.load(x), y, y * ar.qinv));
        } else {
            r = mulmod_b(x, b[i], q, ratio[start + l]);
        }
        break;
    default: r = x ? q - x : 0; break;
    }
    out[i] = r;
}

__global__ void __launch_bounds__(kThreads)
k_from_signed(const int64_t *in, uint64_t *out, const uint64_t *mod, uint32_t start, uint32_t N) {
    const uint32_t l = blockIdx.y, n = blockIdx.x * kThreads + threadIdx.x;
    const uint64_t q = mod[start + l];
    const int64_t v = in[n];
    uint64_t r;
    if (v >= 0) {
        r = (uint64_t)v % q;
    } else {
        r = (uint64_t)(-(v + 1)) % q;  // |v| - 1, avoids overflow at INT64_MIN
        r = q - 1 - r;                 // q - (|v| mod q), in [0, q)
    }
    out[(size_t)l * N + n] = r;
}

// tensor_prod_2x2_rns_poly (src/polymath.cu:463-498), each residue by
// tensor_elem.  Member z = blockIdx.z of a batch reads a, b at + z in_stride
// and writes d0, d1 at + z d_stride, d2 at + z d2_stride.  Each thread takes
// kTensorE elements in pairs of adjacent ones (16-byte accesses); the prime and
// its Barrett ratio are scalar loads.
constexpr int kTensorE = 4;  // elements per thread, in 16-byte pairs

__global__ void __launch_bounds__(kThreads)
k_tensor(const uint64_t *a, const uint64_t *b, uint64_t *d0, uint64_t *d1, uint64_t *d2, const uint64_t *mod,
         const ulonglong2 *ratio, uint32_t Ql, uint32_t N, uint64_t in_stride, uint64_t d_stride,
         uint64_t d2_stride) {
    constexpr int P = kTensorE / 2;
    const uint32_t l = blockIdx.y;
    const uint64_t q = ld_const(mod + l);
    const size_t LN = (size_t)Ql * N, i = (size_t)l * N + (size_t)blockIdx.x * kThreads * kTensorE + threadIdx.x * 2;
    a += blockIdx.z * in_stride;
    b += blockIdx.z * in_stride;
    d0 += blockIdx.z * d_stride;
    d1 += blockIdx.z * d_stride;
    d2 += blockIdx.z * d2_stride;
    // pair p of this thread: elements i + 2 kThreads p, +1 (each pair load is one
    // coalesced 1 KiB row per wave)
    u64x2 a0[P], a1[P], b0[P], b1[P];
#pragma unroll
    for (int p = 0; p < P; p++) {
        const size_t j = i + (size_t)2 * kThreads * p;
        a0[p] = ld_stream2(&a[j]);
        a1[p] = ld_stream2(&a[LN + j]);
        b0[p] = ld_stream2(&b[j]);
        b1[p] = ld_stream2(&b[LN + j]);
    }
    uint64_t r0[kTensorE], r1[kTensorE], r2[kTensorE];
    if (q < kF64PrimeBound) {
        const ArithF64 ar(q);
#pragma unroll
        for (int e = 0; e < kTensorE; e++) {
            const int p = e / 2, h = e % 2;
            tensor_elem(ar, a0[p][h], a1[p][h], b0[p][h], b1[p][h], r0[e], r1[e], r2[e]);
        }
    } else {
        const ulonglong2 r = ld_const(ratio + l);
#pragma unroll
        for (int e = 0; e < kTensorE; e++) {
            const int p = e / 2, h = e % 2;
            tensor_elem(q, r, a0[p][h], a1[p][h], b0[p][h], b1[p][h], r0[e], r1[e], r2[e]);
        }
    }
#pragma unroll
    for (int p = 0; p < P; p++) {
        const size_t j = i + (size_t)2 * kThreads * p;
        st_stream2(&d0[j], r0[2 * p], r0[2 * p + 1]);
        st_stream2(&d1[j], r1[2 * p], r1[2 * p + 1]);
        st_stream2(&d2[j], r2[2 * p], r2[2 * p + 1]);
    }
}

// ModUp base conversion per digit (src/rns_bconv.cu:455-485, :522-528, :530-628):
// slab b, position r of the QlP basis:
//   own limbs (r in digit b): copy of c2 (NTT form)
//   others: y = sum_{i in digit b} t_i [Q_b / q_i]_{p_r}  mod p_r (uncorrected)
// where t = INTT(c2) * [(Q_b / q_i)^-1]_{q_i} (coefficient form, canonical).
__global__ void __launch_bounds__(kThreads)
k_modup_bconv(const uint64_t *t, const uint64_t *c2, uint64_t *out, const uint64_t *mat, const uint64_t *mod,
              const ulonglong2 *ratio, uint32_t Ql, uint32_t alpha, uint32_t Q, uint32_t N) {
    const uint32_t b = blockIdx.y, n = blockIdx.x * kThreads + threadIdx.x;
    const uint32_t QlP = Ql + alpha, st = b * alpha, sz = min(alpha, Ql - st);
    uint64_t tv[kMaxAlpha];
#pragma unroll
    for (uint32_t i = 0; i < kMaxAlpha; i++)
        if (i < sz) tv[i] = t[(size_t)(st + i) * N + n];
    uint64_t *slab = out + (size_t)b * QlP * N;
    const uint64_t *m = mat + (size_t)b * alpha * QlP;
    for (uint32_t r = 0; r < QlP; r++) {
        const size_t o = (size_t)r * N + n;
        if (r >= st && r < st + sz) {
            slab[o] = c2[o];
            continue;
        }
        const uint32_t row = r < Ql ? r : Q + (r - Ql);
        U128 acc{0, 0};
#pragma unroll
        for (uint32_t i = 0; i < kMaxAlpha; i++)
            if (i < sz) mac(acc, tv[i], m[(size_t)i * QlP + r]);
        slab[o] = barrett128(acc, mod[row], ratio[row].x, ratio[row].y);
    }
}

// key_switch_inner_prod_c2_and_evk (src/eval_key_switch.cu:175-230):
//   cx[k][r] = sum_{b < beta} t[b][r] * key[b][k][row(r)]  mod q_row(r)
// accumulated in 128 bits, folded to its residue every 32 digits (a residue
// plus 32 products below 2^122 stays below 2^128; the reference folds at a
// threshold derived from the prime sizes) and reduced at the end: the same
// residues as reducing once.
__global__ void __launch_bounds__(kThreads)
k_ks_inner(const uint64_t *t, const uint64_t *key, uint64_t *cx, const uint64_t *mod, const ulonglong2 *ratio,
           uint32_t Ql, uint32_t QlP, uint32_t Q, uint32_t QP, uint32_t beta, uint32_t N) {
    const uint32_t r = blockIdx.y, n = blockIdx.x * kThreads + threadIdx.x;
    const uint32_t row = r < Ql ? r : Q + (r - Ql);
    const uint64_t q = mod[row];
    const ulonglong2 rt = ratio[row];
    U128 a0{0, 0}, a1{0, 0};
    for (uint32_t b = 0; b < beta; b++) {
        const uint64_t x = t[((size_t)b * QlP + r) * N + n];
        const uint64_t *kb = key + (size_t)b * 2 * QP * N + (size_t)row * N + n;
        mac(a0, x, ld_stream(&kb[0]));
        mac(a1, x, ld_stream(&kb[(size_t)QP * N]));
        if ((b & 31u) == 31u) {
            a0 = U128{barrett128(a0, q, rt.x, rt.y), 0};
            a1 = U128{barrett128(a1, q, rt.x, rt.y), 0};
        }
    }
    uint64_t v0 = barrett128(a0, q, rt.x, rt.y), v1 = barrett128(a1, q, rt.x, rt.y);
    uint64_t *o0 = cx + (size_t)r * N + n, *o1 = cx + ((size_t)QlP + r) * N + n;
    *o0 = v0;
    *o1 = v1;
}

struct Bases {
    const uint64_t *p[2];
};

// apply_galois_ntt_permutation (src/galois.cu:11-18): dst[l][i] = src[l][pi(i)]
__global__ void __launch_bounds__(kThreads)
k_galois(const uint64_t *src, uint64_t *dst, uint32_t elt, uint32_t N, uint32_t logN) {
    const uint32_t l = blockIdx.y, n = blockIdx.x * kThreads + threadIdx.x;
    dst[(size_t)l * N + n] = src[(size_t)l * N + galois_perm(elt, n, logN)];
}

// The inner products of up to m hoisted rotations in one launch (the loop of
// src/evaluate.cu:2036-2050, one rotation per member e):
//   cx_e[k][r] = sum_b t[b][r][sigma_e(n)] key_e[b][k][row(r)][n]  mod q_row(r)
// with the sums of k_ks_inner (folded every 32 digits).  With sum set the
// members' products go into one output, cx_0 (hoisting accumulates the inner
// products of all rotations before one ModDown, src/evaluate.cu:1836-1879):
// the same residues as adding the members' reduced sums.
// Every member reads limb t[b][r] through its own permutation, so the work is
// dealt so that those reads meet in one L2: an item is (target r, half h of
// its positions, block of 256 positions), and the blocks of one (r, h) run on
// workgroups congruent mod 8, i.e. on one XCD (a launch's workgroups are dealt
// to the XCDs round-robin), each XCD taking its pairs (r, h) in turn.
// elts and keys are device tables of m entries.  Digit b's own limbs
// (r in [b alpha, b alpha + alpha), r < Ql) are read from own, the rotated
// ciphertext's c1 in NTT form, and t holds the other (digit, limb) pairs.
__global__ void __launch_bounds__(kThreads)
k_ks_inner_hoist(const uint64_t *t, const uint64_t *own, const uint32_t *elts, const uint64_t *const *keys,
                 uint32_t m, uint32_t sum, uint64_t *cx, uint64_t cx_stride, const uint64_t *mod,
                 const ulonglong2 *ratio, uint32_t Ql, uint32_t QlP, uint32_t Q, uint32_t QP, uint32_t alpha,
                 uint32_t beta, uint32_t N, uint32_t logN) {
    const uint32_t bph = N / kThreads / 2;  // blocks per half of a limb
    const uint32_t jj = blockIdx.x / 8;
    const uint32_t p = (jj / bph) * 8 + blockIdx.x % 8;
    if (p >= 2 * QlP) return;
    const uint32_t r = p >> 1;
    const uint32_t n = ((p & 1) * bph + jj % bph) * kThreads + threadIdx.x;
    const uint32_t row = r < Ql ? r : Q + (r - Ql);
    const uint64_t q = mod[row];
    const ulonglong2 rt = ratio[row];
    const uint64_t *tr = t + (size_t)r * N;
    U128 a0{0, 0}, a1{0, 0};
    uint32_t terms = 0;
    for (uint32_t e = 0; e < m; e++) {
        const uint32_t sn = galois_perm(ld_const(elts + e), n, logN);
        const uint64_t *kr = reinterpret_cast<const uint64_t *>(ld_const(reinterpret_cast<const uint64_t *>(keys + e))) +
                             (size_t)row * N + n;
        for (uint32_t b = 0; b < beta; b++) {
            const uint64_t *src = r < Ql && r / alpha == b ? own + (size_t)r * N : tr + (size_t)b * QlP * N;
            const uint64_t x = src[sn];
            const uint64_t *kb = kr + (size_t)b * 2 * QP * N;
            mac(a0, x, ld_stream(&kb[0]));
            mac(a1, x, ld_stream(&kb[(size_t)QP * N]));
            if (++terms == 32) {
                a0 = U128{barrett128(a0, q, rt.x, rt.y), 0};
                a1 = U128{barrett128(a1, q, rt.x, rt.y), 0};
                terms = 0;
            }
        }
        if (!sum || e + 1 == m) {
            uint64_t *o = cx + (sum ? 0 : (size_t)e * cx_stride) + (size_t)r * N + n;
            o[0] = barrett128(a0, q, rt.x, rt.y);
            o[(size_t)QlP * N] = barrett128(a1, q, rt.x, rt.y);
            a0 = a1 = U128{0, 0};
            terms = 0;
        }
    }
}

// sigma_e(src) for m members (dst_e = dst + e dst_stride), or with sum set
// their sum into dst: the Galois permutation of each hoisted rotation's c0
// (src/galois.cu:11-18), in one launch.
__global__ void __launch_bounds__(kThreads)
k_galois_hoist(const uint64_t *src, uint64_t *dst, uint64_t dst_stride, const uint32_t *elts, uint32_t m,
               uint32_t sum, const uint64_t *mod, uint32_t N, uint32_t logN) {
    const uint32_t l = blockIdx.y, n = blockIdx.x * kThreads + threadIdx.x;
    const uint64_t *sl = src + (size_t)l * N;
    if (sum) {
        const uint64_t q = mod[l];
        uint64_t acc = 0;
        for (uint32_t e = 0; e < m; e++) acc = add_mod(acc, sl[galois_perm(ld_const(elts + e), n, logN)], q);
        dst[(size_t)l * N + n] = acc;
        return;
    }
    const uint32_t e = blockIdx.z;
    dst[(size_t)e * dst_stride + (size_t)l * N + n] = sl[galois_perm(ld_const(elts + e), n, logN)];
}

// generate_one_kswitch_key (src/secretkey.cu:354-398) with
// multiply_temp_mod_and_add_rns_poly (src/polymath.cu:318-336):
//   key[d][0][j] = -(a_d s + e_d)_j + [P]_{q_j} new_key_j * [j in digit d],  key[d][1][j] = a_d
__global__ void __launch_bounds__(kThreads)
k_kswitch_key(const uint64_t *new_key, const uint64_t *s, const uint64_t *a, const uint64_t *e, uint64_t *key,
              const uint64_t *mod, const ulonglong2 *ratio, const ulonglong2 *pmodq, uint32_t QP, uint32_t alpha,
              uint32_t N) {
    const uint32_t j = blockIdx.y, d = blockIdx.z, n = blockIdx.x * kThreads + threadIdx.x;
    const uint64_t q = mod[j];
    const size_t ij = (size_t)j * N + n, idj = ((size_t)d * QP + j) * N + n;
    const uint64_t av = a[idj];
    U128 acc{0, 0};
    mac(acc, av, s[ij]);
    const uint64_t ev = e[idj];
    acc.lo += ev;
    acc.hi += acc.lo < ev ? 1 : 0;
    const uint64_t red = barrett128(acc, q, ratio[j].x, ratio[j].y);
    uint64_t v = red ? q - red : 0;
    if (j >= d * alpha && j < (d + 1) * alpha) v = add_mod(v, shoup(new_key[ij], pmodq[j].x, pmodq[j].y, q), q);
    key[((size_t)d * 2 * QP + j) * N + n] = v;
    key[(((size_t)d * 2 + 1) * QP + j) * N + n] = av;
}

// ------------------------------------------------------------ host helpers
inline dim3 grid(const Ctx &c, uint32_t y, uint32_t z = 1) { return dim3(c.N / kThreads, y, z); }

void check_chain(const Ctx &c, size_t chain) {
    require(chain >= 1 && chain <= c.Q, "chain index out of range (key level 0 is not a data level)");
}

void check_alpha(const Ctx &c) { require(c.P <= kMaxAlpha, "at most 16 special primes are supported"); }

}  // namespace

// ------------------------------------------------------------ operations
// Each takes device pointers and enqueues work on stream s.

void op_modup(const Ctx &c, uint32_t chain, const uint64_t *c2, uint64_t *out, hipStream_t s) {
    check_chain(c, chain);
    check_alpha(c);
    const Level &lv = c.level(chain);
    const uint32_t Ql = lv.Ql, alpha = c.P, QlP = Ql + alpha;
    Scratch sc(c, s);
    uint64_t *t = sc.alloc((size_t)Ql * c.N);
    NttLaunch inv{c2, t, 0, 0, 1, Ql};
    inv.scale = lv.modup_scale;
    ntt_inverse(c, inv, s);
    hipLaunchKernelGGL(k_modup_bconv, grid(c, lv.beta), dim3(kThreads), 0, s, t, c2, out, lv.modup_mat, c.mod,
                       c.ratio, Ql, alpha, c.Q, c.N);
    PFA_HIP(hipGetLastError());
    // NTT every slab except its own digit's limbs (ntt_modup.cu:670-717)
    NttLaunch fw{out, out, (uint64_t)QlP * c.N, (uint64_t)QlP * c.N, lv.beta, QlP};
    fw.start = 0;
    fw.split = Ql;
    fw.split_base = c.Q;
    fw.ex_lo = 0;
    fw.ex_step = alpha;
    fw.ex_len = alpha;
    fw.ex_cap = Ql;
    ntt_forward(c, fw, s);
}

void op_inner(const Ctx &c, uint32_t chain, const uint64_t *t, const uint64_t *key, size_t dnum, uint64_t *cx,
              hipStream_t s) {
    check_chain(c, chain);
    const Level &lv = c.level(chain);
    require(key != nullptr, "null key");
    require(lv.beta <= dnum, "key has fewer digits than the ciphertext level needs");
    const uint32_t QlP = lv.Ql + c.P;
    hipLaunchKernelGGL(k_ks_inner, grid(c, QlP), dim3(kThreads), 0, s, t, key, cx, c.mod, c.ratio, lv.Ql, QlP, c.Q,
                       c.QP, lv.beta, c.N);
    PFA_HIP(hipGetLastError());
}

// The c0 permutations and key inner products of m hoisted rotations of ct
// (ModUp output mu, [beta][QlP][N], each digit's own limbs taken from ct's
// c1): sigma_e(c0) into c0out + e c0_stride and
// member e's inner product into cx + e cx_stride, or with sum set the sum of
// the permuted c0 into c0out and of the inner products into cx.  elts and keys
// are device tables of m entries.
void hoist_inner(const Ctx &c, uint32_t chain, const uint64_t *ct, const uint64_t *mu, const uint32_t *elts,
                 const uint64_t *const *keys, size_t key_dnum, uint32_t m, bool sum, uint64_t *c0out,
                 uint64_t c0_stride, uint64_t *cx, uint64_t cx_stride, hipStream_t s) {
    const Level &lv = c.level(chain);
    require(lv.beta <= key_dnum, "key has fewer digits than the ciphertext level needs");
    const uint32_t Ql = lv.Ql, QlP = Ql + c.P;
    hipLaunchKernelGGL(k_galois_hoist, dim3(c.N / kThreads, Ql, sum ? 1 : m), dim3(kThreads), 0, s, ct, c0out,
                       c0_stride, elts, m, sum ? 1u : 0u, c.mod, c.N, c.logN);
    PFA_HIP(hipGetLastError());
    const uint32_t pairs8 = (2 * QlP + 7) / 8 * 8, bph = c.N / kThreads / 2;
    hipLaunchKernelGGL(k_ks_inner_hoist, dim3(pairs8 * bph), dim3(kThreads), 0, s, mu, ct + (size_t)Ql * c.N, elts,
                       keys, m, sum ? 1u : 0u, cx, cx_stride, c.mod, c.ratio, Ql, QlP, c.Q, c.QP, c.P, lv.beta, c.N,
                       c.logN);
    PFA_HIP(hipGetLastError());
}

// cx [M][QlP][N] -> out [M][Ql][N] (+ base[m] when given), M <= 2
void op_moddown(const Ctx &c, uint32_t chain, const uint64_t *cx, uint32_t M, uint64_t *out, Bases base,
                hipStream_t s) {
    check_chain(c, chain);
    fused_moddown(c, chain, cx, M, out, base.p[0], M > 1 ? base.p[1] : nullptr, s);
}

// out[k] = base_k + KS(c2)_k for k = 0, 1 (out [2][Ql][N]; bases may alias out or be null).
// With count > 1, member i switches c2 + i c2_stride into out + i 2 Ql N with
// bases + i base_stride (the same key).
// With c2_mid (from tensor_for_ks), the ModUp's INTT starts from it.
void op_keyswitch(const Ctx &c, uint32_t chain, const uint64_t *c2, const uint64_t *key, size_t dnum, uint64_t *out,
                  Bases base, hipStream_t s, uint32_t count = 1, uint64_t c2_stride = 0, uint64_t base_stride = 0,
                  const uint64_t *c2_mid = nullptr) {
    check_chain(c, chain);
    const Level &lv = c.level(chain);
    require(key != nullptr, "null key");
    require(lv.beta <= dnum, "key has fewer digits than the ciphertext level needs");
    Scratch sc(c, s);
    const uint64_t cxs = (uint64_t)2 * (lv.Ql + c.P) * c.N;
    uint64_t *cx = sc.alloc((size_t)count * cxs);
    fused_modup_inner(c, chain, c2, key, cx, s, count, c2_stride, cxs, nullptr, nullptr, c2_mid);
    fused_moddown(c, chain, cx, 2 * count, out, base.p[0], base.p[1], s, base_stride);
}

// out [2][Ql-1][N] = rescale(base + KS(c2)): bit-identical to op_keyswitch
// followed by op_rescale, without forming the key-switched ciphertext.  With
// count > 1, member i: c2 + i c2_stride, bases + i base_stride, out + i 2 (Ql-1) N.
void op_keyswitch_rescale(const Ctx &c, uint32_t chain, const uint64_t *c2, const uint64_t *key, size_t dnum,
                          const uint64_t *base0, const uint64_t *base1, uint64_t *out, hipStream_t s,
                          uint32_t count = 1, uint64_t c2_stride = 0, uint64_t base_stride = 0,
                          const uint64_t *c2_mid = nullptr) {
    check_chain(c, chain);
    const Level &lv = c.level(chain);
    require(key != nullptr, "null key");
    require(lv.beta <= dnum, "key has fewer digits than the ciphertext level needs");
    require(lv.Ql >= 2, "cannot rescale at the last level");
    Scratch sc(c, s);
    const uint64_t cxs = (uint64_t)2 * (lv.Ql + c.P) * c.N;
    uint64_t *cx = sc.alloc((size_t)count * cxs);
    const KsFold fold{base0, base1, base_stride};
    fused_modup_inner(c, chain, c2, key, cx, s, count, c2_stride, cxs, &fold, nullptr, c2_mid);
    fused_moddown_rescale(c, chain, cx, base0, base1, out, s, count, base_stride);
}

// count independent products: member i reads a, b at + i in_stride and writes
// d0, d1 at + i d_stride, d2 at + i d2_stride
void op_tensor(const Ctx &c, uint32_t chain, const uint64_t *a, const uint64_t *b, uint64_t *d0, uint64_t *d1,
               uint64_t *d2, hipStream_t s, uint32_t count = 1, uint64_t in_stride = 0, uint64_t d_stride = 0,
               uint64_t d2_stride = 0) {
    check_chain(c, chain);
    const uint32_t Ql = c.size_Ql(chain);
    require(c.N % (kThreads * kTensorE) == 0, "poly_modulus_degree too small for the tensor kernel");
    require(((uintptr_t)a | (uintptr_t)b | (uintptr_t)d0 | (uintptr_t)d1 | (uintptr_t)d2) % 16 == 0 &&
                (in_stride | d_stride | d2_stride) % 2 == 0,
            "tensor operands must be 16-byte aligned");
    hipLaunchKernelGGL(k_tensor, dim3(c.N / (kThreads * kTensorE), Ql, count), dim3(kThreads), 0, s, a, b, d0, d1, d2,
                       c.mod, c.ratio, Ql, c.N, in_stride, d_stride, d2_stride);
    PFA_HIP(hipGetLastError());
}

// op_tensor for a product whose d2 is key-switched next: at N <= 2^16 the
// tensor kernel also runs the first pass of the key switch's INTT(d2) and the
// returned buffer (count x Ql N, from sc) holds it for op_keyswitch /
// op_keyswitch_rescale; otherwise plain op_tensor
// and nullptr.
const uint64_t *tensor_for_ks(const Ctx &c, Scratch &sc, uint32_t chain, const uint64_t *a, const uint64_t *b,
                              uint64_t *d0, uint64_t *d1, uint64_t *d2, hipStream_t s, uint32_t count = 1,
                              uint64_t in_stride = 0, uint64_t d_stride = 0, uint64_t d2_stride = 0) {
    if (c.logN > 16) {
        op_tensor(c, chain, a, b, d0, d1, d2, s, count, in_stride, d_stride, d2_stride);
        return nullptr;
    }
    check_chain(c, chain);
    uint64_t *mid = sc.alloc((size_t)count * c.size_Ql(chain) * c.N);
    fused_tensor_rows(c, chain, a, b, d0, d1, d2, mid, s, count, in_stride, d_stride, d2_stride);
    return mid;
}

void op_galois(const Ctx &c, uint32_t elt, const uint64_t *src, uint64_t *dst, uint32_t L, hipStream_t s) {
    require((elt & 1) && elt < 2 * c.N, "Galois element must be odd and below 2N");
    require(src != dst, "apply_galois_ntt cannot run in place");
    hipLaunchKernelGGL(k_galois, grid(c, L), dim3(kThreads), 0, s, src, dst, elt, c.N, c.logN);
    PFA_HIP(hipGetLastError());
}

void op_rescale(const Ctx &c, uint32_t chain, const uint64_t *in, uint32_t size, uint64_t *out, hipStream_t s) {
    check_chain(c, chain);
    require(c.level(chain).Ql >= 2, "cannot rescale at the last level");
    require(size >= 1 && size <= 65535, "bad ciphertext size");
    fused_rescale(c, chain, in, size, out, s);
}

}  // namespace pfa

using namespace pfa;

extern "C" {

int pfa_modup(const pfa_context *ctx, size_t chain_index, const uint64_t *c2, uint64_t *t_mod_up, void *stream) {
    return guarded([&] {
        require(c2 && t_mod_up, "null argument");
        op_modup(*ctx_of(ctx), (uint32_t)chain_index, c2, t_mod_up, as_stream(stream));
    });
}

int pfa_ks_inner_prod(const pfa_context *ctx, size_t chain_index, const uint64_t *t_mod_up, const uint64_t *key,
                      size_t key_dnum, uint64_t *cx, void *stream) {
    return guarded([&] {
        require(t_mod_up && cx, "null argument");
        op_inner(*ctx_of(ctx), (uint32_t)chain_index, t_mod_up, key, key_dnum, cx, as_stream(stream));
    });
}

int pfa_moddown(const pfa_context *ctx, size_t chain_index, const uint64_t *cx_k, uint64_t *out, void *stream) {
    return guarded([&] {
        require(cx_k && out, "null argument");
        op_moddown(*ctx_of(ctx), (uint32_t)chain_index, cx_k, 1, out, Bases{{nullptr, nullptr}}, as_stream(stream));
    });
}

int pfa_keyswitch(const pfa_context *ctx, size_t chain_index, uint64_t *ct, const uint64_t *c2, const uint64_t *key,
                  size_t key_dnum, void *stream) {
    return guarded([&] {
        const Ctx &c = *ctx_of(ctx);
        require(ct && c2, "null argument");
        check_chain(c, chain_index);
        const size_t LN = (size_t)c.size_Ql((uint32_t)chain_index) * c.N;
        op_keyswitch(c, (uint32_t)chain_index, c2, key, key_dnum, ct, Bases{{ct, ct + LN}}, as_stream(stream));
    });
}

int pfa_tensor(const pfa_context *ctx, size_t chain_index, const uint64_t *a, const uint64_t *b, uint64_t *out,
               void *stream) {
    return guarded([&] {
        const Ctx &c = *ctx_of(ctx);
        require(a && b && out, "null argument");
        check_chain(c, chain_index);
        const size_t LN = (size_t)c.size_Ql((uint32_t)chain_index) * c.N;
        op_tensor(c, (uint32_t)chain_index, a, b, out, out + LN, out + 2 * LN, as_stream(stream));
    });
}

int pfa_multiply_and_relin(const pfa_context *ctx, size_t chain_index, const uint64_t *a, const uint64_t *b,
                           const uint64_t *rlk, size_t key_dnum, uint64_t *out, void *stream) {
    return guarded([&] {
        const Ctx &c = *ctx_of(ctx);
        require(a && b && out && rlk, "null argument");
        check_chain(c, chain_index);
        const hipStream_t s = as_stream(stream);
        const size_t LN = (size_t)c.size_Ql((uint32_t)chain_index) * c.N;
        Scratch sc(c, s);
        uint64_t *c2 = sc.alloc(LN);
        const uint64_t *mid = tensor_for_ks(c, sc, (uint32_t)chain_index, a, b, out, out + LN, c2, s);
        op_keyswitch(c, (uint32_t)chain_index, c2, rlk, key_dnum, out, Bases{{out, out + LN}}, s, 1, 0, 0, mid);
    });
}

int pfa_relinearize(const pfa_context *ctx, size_t chain_index, const uint64_t *ct3, const uint64_t *rlk,
                    size_t key_dnum, uint64_t *out, void *stream) {
    return guarded([&] {
        const Ctx &c = *ctx_of(ctx);
        require(ct3 && out && rlk, "null argument");
        check_chain(c, chain_index);
        const size_t LN = (size_t)c.size_Ql((uint32_t)chain_index) * c.N;
        op_keyswitch(c, (uint32_t)chain_index, ct3 + 2 * LN, rlk, key_dnum, out, Bases{{ct3, ct3 + LN}},
                     as_stream(stream));
    });
}

int pfa_multiply_relin_rescale(const pfa_context *ctx, size_t chain_index, const uint64_t *a, const uint64_t *b,
                               const uint64_t *rlk, size_t key_dnum, uint64_t *out, void *stream) {
    return guarded([&] {
        const Ctx &c = *ctx_of(ctx);
        require(a && b && out && rlk, "null argument");
        require(out != a && out != b, "output must not alias an input");
        check_chain(c, chain_index);
        require(c.size_Ql((uint32_t)chain_index) >= 2, "cannot rescale at the last level");
        const hipStream_t s = as_stream(stream);
        const size_t LN = (size_t)c.size_Ql((uint32_t)chain_index) * c.N;
        Scratch sc(c, s);
        uint64_t *d = sc.alloc(3 * LN);
        const uint64_t *mid = tensor_for_ks(c, sc, (uint32_t)chain_index, a, b, d, d + LN, d + 2 * LN, s);
        op_keyswitch_rescale(c, (uint32_t)chain_index, d + 2 * LN, rlk, key_dnum, d, d + LN, out, s, 1, 0, 0, mid);
    });
}

int pfa_multiply_and_relin_batch(const pfa_context *ctx, size_t chain_index, size_t count, const uint64_t *a,
                                 const uint64_t *b, const uint64_t *rlk, size_t key_dnum, uint64_t *out,
                                 void *stream) {
    return guarded([&] {
        const Ctx &c = *ctx_of(ctx);
        require(a && b && out && rlk, "null argument");
        require(count >= 1 && count <= 4096, "count out of range");
        check_chain(c, chain_index);
        const hipStream_t s = as_stream(stream);
        const size_t LN = (size_t)c.size_Ql((uint32_t)chain_index) * c.N;
        require(out + count * 2 * LN <= a || out >= a + count * 2 * LN || out == a, "output overlaps an input");
        require(out + count * 2 * LN <= b || out >= b + count * 2 * LN || out == b, "output overlaps an input");
        Scratch sc(c, s);
        uint64_t *c2 = sc.alloc(count * LN);
        // d0, d1 into out (the key switch adds to them in place), d2 of member i to c2 + i LN
        const uint64_t *mid = tensor_for_ks(c, sc, (uint32_t)chain_index, a, b, out, out + LN, c2, s,
                                            (uint32_t)count, 2 * LN, 2 * LN, LN);
        op_keyswitch(c, (uint32_t)chain_index, c2, rlk, key_dnum, out, Bases{{out, out + LN}}, s, (uint32_t)count,
                     LN, 2 * LN, mid);
    });
}

int pfa_multiply_relin_rescale_batch(const pfa_context *ctx, size_t chain_index, size_t count, const uint64_t *a,
                                     const uint64_t *b, const uint64_t *rlk, size_t key_dnum, uint64_t *out,
                                     void *stream) {
    return guarded([&] {
        const Ctx &c = *ctx_of(ctx);
        require(a && b && out && rlk, "null argument");
        require(count >= 1 && count <= 4096, "count out of range");
        check_chain(c, chain_index);
        require(c.size_Ql((uint32_t)chain_index) >= 2, "cannot rescale at the last level");
        const hipStream_t s = as_stream(stream);
        const size_t LN = (size_t)c.size_Ql((uint32_t)chain_index) * c.N, ON = LN - c.N;
        require(out + count * 2 * ON <= a || out >= a + count * 2 * LN, "output overlaps an input");
        require(out + count * 2 * ON <= b || out >= b + count * 2 * LN, "output overlaps an input");
        Scratch sc(c, s);
        // member i: d0, d1, d2 at d + i 3 LN
        uint64_t *d = sc.alloc(count * 3 * LN);
        const uint64_t *mid = tensor_for_ks(c, sc, (uint32_t)chain_index, a, b, d, d + LN, d + 2 * LN, s,
                                            (uint32_t)count, 2 * LN, 3 * LN, 3 * LN);
        op_keyswitch_rescale(c, (uint32_t)chain_index, d + 2 * LN, rlk, key_dnum, d, d + LN, out, s, (uint32_t)count,
                             3 * LN, 3 * LN, mid);
    });
}

int pfa_relinearize_rescale(const pfa_context *ctx, size_t chain_index, const uint64_t *ct3, const uint64_t *rlk,
                            size_t key_dnum, uint64_t *out, void *stream) {
    return guarded([&] {
        const Ctx &c = *ctx_of(ctx);
        require(ct3 && out && rlk, "null argument");
        require(out != ct3, "output must not alias the input");
        check_chain(c, chain_index);
        const size_t LN = (size_t)c.size_Ql((uint32_t)chain_index) * c.N;
        op_keyswitch_rescale(c, (uint32_t)chain_index, ct3 + 2 * LN, rlk, key_dnum, ct3, ct3 + LN, out,
                             as_stream(stream));
    });
}

int pfa_rescale(const pfa_context *ctx, size_t chain_index, const uint64_t *in, size_t size, uint64_t *out,
                void *stream) {
    return guarded([&] {
        require(in && out && in != out, "rescale needs distinct input and output buffers");
        op_rescale(*ctx_of(ctx), (uint32_t)chain_index, in, (uint32_t)size, out, as_stream(stream));
    });
}

int pfa_galois_elt_from_step(int step, uint64_t poly_degree, uint32_t *elt) {
    return guarded([&] {
        require(elt != nullptr, "null argument");
        require(poly_degree >= 2 && (poly_degree & (poly_degree - 1)) == 0 && poly_degree <= (1u << 30),
                "poly_modulus_degree must be a power of two");
        // get_elt_from_step (include/galois.cuh:16-49)
        const uint64_t n = poly_degree, m = 2 * n;
        if (step == 0) {
            *elt = (uint32_t)(m - 1);
            return;
        }
        const uint64_t pos = step < 0 ? (uint64_t)(-(int64_t)step) : (uint64_t)step;
        require(pos < n / 2, "step count too large");
        uint64_t k = step < 0 ? n / 2 - pos : pos;
        uint64_t g = 1;
        while (k--) g = (g * 5) & (m - 1);
        *elt = (uint32_t)g;
    });
}

int pfa_apply_galois_ntt(const pfa_context *ctx, uint32_t elt, const uint64_t *src, uint64_t *dst, size_t L,
                         void *stream) {
    return guarded([&] {
        require(src && dst && L >= 1, "null argument");
        op_galois(*ctx_of(ctx), elt, src, dst, (uint32_t)L, as_stream(stream));
    });
}

int pfa_apply_galois(const pfa_context *ctx, size_t chain_index, uint64_t *ct, uint32_t elt, const uint64_t *key,
                     size_t key_dnum, void *stream) {
    return guarded([&] {
        const Ctx &c = *ctx_of(ctx);
        require(ct && key, "null argument");
        check_chain(c, chain_index);
        const hipStream_t s = as_stream(stream);
        const uint32_t Ql = c.size_Ql((uint32_t)chain_index);
        const size_t LN = (size_t)Ql * c.N;
        Scratch sc(c, s);
        uint64_t *t = sc.alloc(2 * LN);
        // c0' = sigma(c0) + KS0(sigma(c1)), c1' = KS1(sigma(c1))  (src/evaluate.cu:1607-1656)
        if (c.logN <= 16) {
            // the permutation kernel also runs the first pass of the key switch's INTT
            uint64_t *mid = sc.alloc(LN);
            galois_rows(c, (uint32_t)chain_index, ct, 0, 1, elt, nullptr, nullptr, t, mid, s);
            op_keyswitch(c, (uint32_t)chain_index, t + LN, key, key_dnum, ct, Bases{{t, nullptr}}, s, 1, 0, 0, mid);
        } else {
            op_galois(c, elt, ct, t, Ql, s);
            op_galois(c, elt, ct + LN, t + LN, Ql, s);
            op_keyswitch(c, (uint32_t)chain_index, t + LN, key, key_dnum, ct, Bases{{t, nullptr}}, s);
        }
    });
}

int pfa_hoist_rotations(const pfa_context *ctx, size_t chain_index, const uint64_t *ct, const uint32_t *elts,
                        size_t n, const uint64_t *const *keys, size_t key_dnum, uint64_t *out, void *stream) {
    return guarded([&] {
        const Ctx &c = *ctx_of(ctx);
        require(ct && out && (n == 0 || (elts && keys)), "null argument");
        check_chain(c, chain_index);
        if (n == 0) return;
        const hipStream_t s = as_stream(stream);
        const uint32_t chain = (uint32_t)chain_index;
        const Level &lv = c.level(chain);
        const uint32_t Ql = lv.Ql, QlP = Ql + c.P;
        const size_t LN = (size_t)Ql * c.N;
        for (size_t e = 0; e < n; ++e) require((elts[e] & 1) && elts[e] < 2 * c.N, "bad Galois element");
        Scratch sc(c, s);
        uint64_t *mu = sc.alloc((size_t)lv.beta * QlP * c.N);
        fused_modup_ntt(c, chain, ct + LN, mu, s);
        // up to kHoistGroup rotations at a time: their c0 permutations (into
        // poly 0 of each output) and inner products (each into its own slot)
        // in one launch each, then one ModDown over the group's 2 m polys
        // (its small INTT and base-conversion launches are latency-bound, so
        // one launch for the group costs about what one rotation's did), poly
        // 2e adding sigma_e(c0)
        constexpr size_t kHoistGroup = 16;
        const size_t CX = (size_t)2 * QlP * c.N;
        const size_t G = std::min(n, kHoistGroup);
        uint64_t *cx = sc.alloc(G * CX);
        for (size_t e0 = 0; e0 < n; e0 += kHoistGroup) {
            const uint32_t m = (uint32_t)std::min(kHoistGroup, n - e0);
            void *dev[2];
            upload_parts(c, sc, s, {{elts + e0, m * sizeof(uint32_t)}, {keys + e0, m * sizeof(void *)}}, dev);
            const uint32_t *elt_dev = (const uint32_t *)dev[0];
            const uint64_t *const *key_dev = (const uint64_t *const *)dev[1];
            uint64_t *o = out + e0 * 2 * LN;
            hoist_inner(c, chain, ct, mu, elt_dev, key_dev, key_dnum, m, false, o, 2 * LN, cx, CX, s);
            fused_moddown(c, chain, cx, 2 * m, o, o, nullptr, s, 2 * LN);
        }
    });
}

int pfa_hoisting(const pfa_context *ctx, size_t chain_index, const uint64_t *ct, const uint32_t *elts, size_t n,
                 const uint64_t *const *keys, size_t key_dnum, uint64_t *out, void *stream) {
    return guarded([&] {
        const Ctx &c = *ctx_of(ctx);
        require(ct && out && n >= 1 && elts && keys, "null argument or no rotation steps");
        check_chain(c, chain_index);
        const hipStream_t s = as_stream(stream);
        const uint32_t chain = (uint32_t)chain_index;
        const Level &lv = c.level(chain);
        const uint32_t Ql = lv.Ql, QlP = Ql + c.P;
        const size_t LN = (size_t)Ql * c.N;
        for (size_t e = 0; e < n; ++e) require((elts[e] & 1) && elts[e] < 2 * c.N, "bad Galois element");
        Scratch sc(c, s);
        uint64_t *mu = sc.alloc((size_t)lv.beta * QlP * c.N);
        fused_modup_ntt(c, chain, ct + LN, mu, s);
        uint64_t *cx = sc.alloc((size_t)2 * QlP * c.N);
        uint64_t *c0 = sc.alloc(LN);  // sum of sigma_e(c0)
        void *dev[2];
        upload_parts(c, sc, s, {{elts, n * sizeof(uint32_t)}, {keys, n * sizeof(void *)}}, dev);
        hoist_inner(c, chain, ct, mu, (const uint32_t *)dev[0], (const uint64_t *const *)dev[1], key_dnum,
                    (uint32_t)n, true, c0, 0, cx, 0, s);
        // c0' = sum sigma(c0) + ModDown(acc0), c1' = ModDown(acc1)
        op_moddown(c, chain, cx, 2, out, Bases{{c0, nullptr}}, s);
    });
}

int pfa_kswitch_key(const pfa_context *ctx, const uint64_t *new_key, const uint64_t *s_key, const uint64_t *a,
                    const uint64_t *e, uint64_t *key, void *stream) {
    return guarded([&] {
        const Ctx &c = *ctx_of(ctx);
        require(new_key && s_key && a && e && key, "null argument");
        const uint32_t dnum = c.Q / c.P;
        require(dnum >= 1, "need at least one key digit");
        hipLaunchKernelGGL(k_kswitch_key, grid(c, c.QP, dnum), dim3(kThreads), 0, as_stream(stream), new_key, s_key,
                           a, e, key, c.mod, c.ratio, c.pmodq, c.QP, c.P, c.N);
        PFA_HIP(hipGetLastError());
    });
}

static int binop(const pfa_context *ctx, int op, const uint64_t *a, const uint64_t *b, uint64_t *out, size_t L,
                 size_t start, void *stream) {
    return guarded([&] {
        const Ctx &c = *ctx_of(ctx);
        require(a && out && (op == kNeg || b), "null argument");
        require(L >= 1 && start + L <= c.QP, "limb range exceeds the context's primes");
        hipLaunchKernelGGL(k_poly_binop, grid(c, (uint32_t)L), dim3(kThreads), 0, as_stream(stream), op, a,
                           op == kNeg ? a : b, out, c.mod, c.ratio, (uint32_t)start, c.N, 0ull, 0ull, 0ull);
        PFA_HIP(hipGetLastError());
    });
}

int pfa_poly_add(const pfa_context *ctx, const uint64_t *a, const uint64_t *b, uint64_t *out, size_t L, size_t start,
                 void *stream) {
    return binop(ctx, kAdd, a, b, out, L, start, stream);
}
int pfa_poly_sub(const pfa_context *ctx, const uint64_t *a, const uint64_t *b, uint64_t *out, size_t L, size_t start,
                 void *stream) {
    return binop(ctx, kSub, a, b, out, L, start, stream);
}
int pfa_poly_mul(const pfa_context *ctx, const uint64_t *a, const uint64_t *b, uint64_t *out, size_t L, size_t start,
                 void *stream) {
    return binop(ctx, kMul, a, b, out, L, start, stream);
}
int pfa_ct_multiply_plain(const pfa_context *ctx, const uint64_t *ct, size_t size, const uint64_t *pt, uint64_t *out,
                          size_t L, void *stream) {
    return guarded([&] {
        const Ctx &c = *ctx_of(ctx);
        require(ct && pt && out, "null argument");
        require(L >= 1 && L <= c.Q, "limb count out of range");
        require(size >= 1 && size <= 65535, "bad ciphertext size");
        const uint64_t LN = (uint64_t)L * c.N;
        hipLaunchKernelGGL(k_poly_binop, grid(c, (uint32_t)L, (uint32_t)size), dim3(kThreads), 0, as_stream(stream),
                           (int)kMul, ct, pt, out, c.mod, c.ratio, 0u, c.N, LN, 0ull, LN);
        PFA_HIP(hipGetLastError());
    });
}

int pfa_poly_negate(const pfa_context *ctx, const uint64_t *a, uint64_t *out, size_t L, size_t start, void *stream) {
    return binop(ctx, kNeg, a, nullptr, out, L, start, stream);
}

int pfa_poly_from_signed(const pfa_context *ctx, const int64_t *in, uint64_t *out, size_t L, size_t start,
                         void *stream) {
    return guarded([&] {
        const Ctx &c = *ctx_of(ctx);
        require(in && out, "null argument");
        require(L >= 1 && start + L <= c.QP, "limb range exceeds the context's primes");
        hipLaunchKernelGGL(k_from_signed, grid(c, (uint32_t)L), dim3(kThreads), 0, as_stream(stream), in, out, c.mod,
                           (uint32_t)start, c.N);
        PFA_HIP(hipGetLastError());
    });
}

}  // extern "C"
