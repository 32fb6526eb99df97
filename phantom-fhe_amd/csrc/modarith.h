// Device modular arithmetic for the CKKS hot path on gfx950.
//
// Two arithmetic policies share every NTT kernel; the policy is chosen per
// limb from the limb's prime (uniform per workgroup, no divergence):
//
//   ArithF64 -- primes q < 2^50.  Residues live in registers as exact integers
//               held in doubles.  A modular product costs six full-rate FP64
//               VALU ops (two-product split + rounded quotient), against ~20
//               32-bit integer ops for 64-bit Shoup on this ISA.
//   ArithInt -- any prime q < 2^62.  Harvey-style lazy Shoup butterflies on
//               uint64 ([0, 4q) between stages).
//
// Both policies are exact: every butterfly output is congruent mod q to the
// textbook value, and outputs are brought to the canonical range [0, q)
// before they leave a kernel.  Results are therefore bit-identical to the
// reference's (src/ntt/ntt_1d.cu:17-292, include/butterfly.cuh), whose
// kernels also emit canonical residues.
//
// Exactness bounds of ArithF64 (q < 2^50, twiddle w in [0, q), wq = fl(w/q)):
//   mul(y, w) with |y| <= B q, B <= 8:
//     qt = rint(fl(y*wq))          |qt - y w / q| <= 1 + B/16
//     h = fl(y*w), l = fma(y,w,-h)  y w = h + l exactly, |l| <= 2^50
//     r1 = fma(-qt, q, h)           exact: |h - qt q| < 2^52 is an integer
//     r  = r1 + l                   exact, r == y w - qt q, |r| <= (1 + B/16) q
//   A CT butterfly maps bound B to B + 1 + B/16: four stages from B = 1 reach
//   5.66 < 8, so each four-stage round starts from a reduced value
//   (reduce(): |x| <= 1 q after x - rint(x/q) q).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pfa {

constexpr uint64_t kF64PrimeBound = 1ULL << 50;

__device__ __forceinline__ uint64_t mulhi64(uint64_t a, uint64_t b) { return __umul64hi(a, b); }

__device__ __forceinline__ uint64_t csub(uint64_t x, uint64_t q) { return x >= q ? x - q : x; }

// Load of streamed data that is read once (residues of a batch, key limbs):
// the nontemporal hint keeps it from displacing reused lines (twiddle tables,
// shared input tiles) and raises the achieved bandwidth of the NTT passes on
// gfx950 (measured: 2 x 35 limbs at N = 2^16, forward NTT 49.5 -> 38.6 us with
// streaming loads and stores).
__device__ __forceinline__ uint64_t ld_stream(const uint64_t *p) { return __builtin_nontemporal_load(p); }
// Store counterpart for results written once; with both hints the NTT passes
// stream faster than with either alone.
__device__ __forceinline__ void st_stream(uint64_t *p, uint64_t v) { __builtin_nontemporal_store(v, p); }

// y * w mod q in [0, 2q) for any y < 2^64, w < q < 2^63, ws = floor(w 2^64 / q).
__device__ __forceinline__ uint64_t shoup_lazy(uint64_t y, uint64_t w, uint64_t ws, uint64_t q) {
    return y * w - mulhi64(y, ws) * q;
}

__device__ __forceinline__ uint64_t shoup(uint64_t y, uint64_t w, uint64_t ws, uint64_t q) {
    return csub(shoup_lazy(y, w, ws, q), q);
}

__device__ __forceinline__ uint64_t add_mod(uint64_t a, uint64_t b, uint64_t q) { return csub(a + b, q); }

__device__ __forceinline__ uint64_t sub_mod(uint64_t a, uint64_t b, uint64_t q) { return a >= b ? a - b : a + q - b; }

// 128-bit accumulator for sums of products.
struct U128 {
    uint64_t lo, hi;
};

// Full 64 x 64 -> 128-bit product from the four 32 x 32 partial products,
// each one v_mad_u64_u32 (32 x 32 + 64 -> 64); written out because a * b and
// __umul64hi(a, b) separately take 3 + 4 multiplies.  No sum overflows:
// s1, s2 <= (2^32 - 1)^2 + 2^32 - 1 < 2^64 and hi <= (2^32 - 1)^2 + 2 (2^32 - 1).
__device__ __forceinline__ U128 mul_wide(uint64_t a, uint64_t b) {
    const uint64_t a0 = (uint32_t)a, a1 = a >> 32, b0 = (uint32_t)b, b1 = b >> 32;
    const uint64_t p00 = a0 * b0;
    const uint64_t s1 = a1 * b0 + (p00 >> 32);
    const uint64_t s2 = a0 * b1 + (uint32_t)s1;
    return U128{(s2 << 32) | (uint32_t)p00, a1 * b1 + (s1 >> 32) + (s2 >> 32)};
}

__device__ __forceinline__ void mac(U128 &acc, uint64_t a, uint64_t b) {
    const U128 p = mul_wide(a, b);
    acc.lo += p.lo;
    acc.hi += p.hi + (acc.lo < p.lo ? 1 : 0);
}

// x mod q for any 128-bit x, with ratio = floor(2^128 / q) = (r1 : r0).
// The quotient estimate drops only the low word of x0*r0 and the truncation of
// ratio, so it is at most 2 below floor(x/q); two conditional subtractions
// finish (requires 3q < 2^64).
__device__ __forceinline__ uint64_t barrett128(U128 x, uint64_t q, uint64_t r0, uint64_t r1) {
    uint64_t c = mulhi64(x.lo, r0);
    uint64_t a_lo = x.lo * r1, a_hi = mulhi64(x.lo, r1);
    uint64_t s = a_lo + c;
    uint64_t t = a_hi + (s < c ? 1 : 0);
    uint64_t b_lo = x.hi * r0, b_hi = mulhi64(x.hi, r0);
    uint64_t s2 = s + b_lo;
    uint64_t u = b_hi + (s2 < b_lo ? 1 : 0) + t;
    uint64_t est = x.hi * r1 + u;
    uint64_t r = x.lo - est * q;
    r = csub(r, q);
    return csub(r, q);
}

// Montgomery reduction T 2^-64 mod q, in [0, 2q), of a 128-bit T < q 2^64.
__device__ __forceinline__ uint64_t mont_reduce(U128 t, uint64_t q, uint64_t qn) {
    const uint64_t m = t.lo * qn;
    return t.hi + mulhi64(m, q) + (t.lo != 0 ? 1 : 0);
}

// Montgomery product x y 2^-64 mod q, in [0, 2q), for x y < q 2^64 (e.g. x < 4q,
// y < q with q < 2^62); qn = -q^-1 mod 2^64.  With m = lo(x y) qn, x y + m q is
// a multiple of 2^64 whose low word sums to 0 or 2^64 (lo(x y) != 0).
__device__ __forceinline__ uint64_t mont_mul(uint64_t x, uint64_t y, uint64_t q, uint64_t qn) {
    const U128 p = mul_wide(x, y);
    const uint64_t m = p.lo * qn;
    return p.hi + mulhi64(m, q) + (p.lo != 0 ? 1 : 0);
}


// ----------------------------------------------------------------------------
// NTT arithmetic policies.  Twiddle table entries are 16-byte pairs whose
// meaning depends on the prime's policy:
//   ArithInt: (w, floor(w 2^64 / q))
//   ArithF64: (bits of double(w), bits of fl(w / q))
// ----------------------------------------------------------------------------

struct ArithInt {
    using T = uint64_t;
    static constexpr bool kF64 = false;
    uint64_t q, q2;

    __device__ __forceinline__ explicit ArithInt(uint64_t q_) : q(q_), q2(2 * q_) {}

    __device__ __forceinline__ T load(uint64_t v) const { return v; }
    // canonical residue from [0, 4q)
    __device__ __forceinline__ uint64_t store(T v) const { return csub(csub(v, q2), q); }
    // intermediate (between the two passes of one transform): keep lazy form
    __device__ __forceinline__ uint64_t store_mid(T v) const { return v; }
    __device__ __forceinline__ T load_mid(uint64_t v) const { return v; }
    __device__ __forceinline__ void reduce(T &) const {}

    // Cooley-Tukey: (x, y) -> (x + w y, x - w y); inputs and outputs in [0, 4q)
    __device__ __forceinline__ void ct(T &x, T &y, ulonglong2 w) const {
        uint64_t a = csub(x, q2);
        uint64_t t = shoup_lazy(y, w.x, w.y, q);
        x = a + t;
        y = a - t + q2;
    }
    // Gentleman-Sande: (x, y) -> (x + y, (x - y) w); inputs and outputs in [0, 2q)
    __device__ __forceinline__ void gs(T &x, T &y, ulonglong2 w) const {
        uint64_t s = csub(x + y, q2);
        uint64_t d = x - y + q2;
        x = s;
        y = shoup_lazy(d, w.x, w.y, q);
    }
    // last inverse stage: (x, y) -> ((x + y) n, (x - y) w) with n = N^-1 (a pair)
    __device__ __forceinline__ void gs_last(T &x, T &y, ulonglong2 w, ulonglong2 n) const {
        uint64_t s = x + y;
        uint64_t d = x - y + q2;
        x = shoup_lazy(s, n.x, n.y, q);
        y = shoup_lazy(d, w.x, w.y, q);
    }
    __device__ __forceinline__ void mul(T &x, ulonglong2 c) const { x = shoup_lazy(x, c.x, c.y, q); }
};

struct ArithF64 {
    using T = double;
    static constexpr bool kF64 = true;
    double q, qinv;

    __device__ __forceinline__ explicit ArithF64(uint64_t q_) : q((double)q_), qinv(1.0 / (double)q_) {}

    static __device__ __forceinline__ double as_f(uint64_t b) { return __longlong_as_double((long long)b); }
    static __device__ __forceinline__ uint64_t as_u(double d) { return (uint64_t)__double_as_longlong(d); }

    // Integer <-> double through the exponent bias: for 0 <= v < 2^52 the
    // double with bits (0x433 << 52) | v is exactly 2^52 + v.
    static constexpr uint64_t kBias = 0x4330000000000000ull;
    static constexpr double kTwo52 = 4503599627370496.0;
    static constexpr uint64_t kMant = (1ull << 52) - 1;
    // exact for v < 2^52 (every residue of a prime below 2^50)
    __device__ __forceinline__ T load(uint64_t v) const { return as_f(v | kBias) - kTwo52; }
    // canonical residue of any integer-valued |v| < 2^53: with k the nearest
    // integer to fl(v / q), v - k q lies within (0.5 + 2^-19) q of zero (and is
    // computed exactly by the FMA), so one conditional add of q lands in [0, q).
    __device__ __forceinline__ uint64_t store(T v) const {
        const double k = rint(v * qinv);
        double r = __fma_rn(-k, q, v);
        r = r < 0.0 ? r + q : r;
        return as_u(r + kTwo52) & kMant;
    }
    __device__ __forceinline__ uint64_t store_mid(T v) const {
        reduce(v);
        return as_u(v);
    }
    __device__ __forceinline__ T load_mid(uint64_t v) const { return as_f(v); }
    __device__ __forceinline__ void reduce(T &x) const { x = __fma_rn(-rint(x * qinv), q, x); }

    __device__ __forceinline__ T mulw(T y, double w, double wq) const {
        double qt = rint(y * wq);
        double h = y * w;
        double l = __fma_rn(y, w, -h);
        return __fma_rn(-qt, q, h) + l;
    }
    __device__ __forceinline__ void ct(T &x, T &y, ulonglong2 w) const {
        double t = mulw(y, as_f(w.x), as_f(w.y));
        y = x - t;
        x = x + t;
    }
    __device__ __forceinline__ void gs(T &x, T &y, ulonglong2 w) const {
        double s = x + y;
        double d = x - y;
        reduce(s);
        x = s;
        y = mulw(d, as_f(w.x), as_f(w.y));
    }
    __device__ __forceinline__ void gs_last(T &x, T &y, ulonglong2 w, ulonglong2 n) const {
        double s = x + y;
        double d = x - y;
        x = mulw(s, as_f(n.x), as_f(n.y));
        y = mulw(d, as_f(w.x), as_f(w.y));
    }
    __device__ __forceinline__ void mul(T &x, ulonglong2 c) const { x = mulw(x, as_f(c.x), as_f(c.y)); }

    // Twiddle pair of base * s for a table pair `base` and a small-table pair s:
    // w = base w * s w with |w| <= (1 + 1/16) q, and wq = w / q to within half
    // an ulp (one FMA correction step), which keeps the butterfly bound above
    // (growth B -> B + 1 + B/8 per stage, four stages from B = 1 reach 6.4 < 8).
    __device__ __forceinline__ ulonglong2 twmul(ulonglong2 base, ulonglong2 s) const { return pair_of(twval(base, s)); }
    // the twiddle value of twmul alone, and the pair twmul forms from it
    __device__ __forceinline__ double twval(ulonglong2 base, ulonglong2 s) const {
        return mulw(as_f(base.x), as_f(s.x), as_f(s.y));
    }
    __device__ __forceinline__ ulonglong2 pair_of(double w) const {
        double wq = w * qinv;
        const double e = __fma_rn(-wq, q, w);
        wq = __fma_rn(e, qinv, wq);
        return ulonglong2{as_u(w), as_u(wq)};
    }
};

// A value the caller knows to be the same in every lane, moved to scalar
// registers (a load through a pointer the compiler cannot prove read-only
// leaves it in vector registers).
__device__ __forceinline__ uint64_t wave_uniform(uint64_t v) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return ((uint64_t)hi << 32) | lo;
}

// Loads of read-only tables at a wave-uniform index, issued as scalar loads
// (constant address space): counted by lgkmcnt, so a kernel that has
// prefetched its next tile's residues can read them without waiting for the
// prefetch (vector loads complete in issue order).
__device__ __forceinline__ uint64_t ld_const(const uint64_t *p) {
    return *(const __attribute__((address_space(4))) uint64_t *)p;
}
__device__ __forceinline__ uint32_t ld_const(const uint32_t *p) {
    return *(const __attribute__((address_space(4))) uint32_t *)p;
}
__device__ __forceinline__ ulonglong2 ld_const(const ulonglong2 *p) {
    const uint64_t *w = reinterpret_cast<const uint64_t *>(p);
    return ulonglong2{ld_const(w), ld_const(w + 1)};
}
__device__ __forceinline__ uint32_t uniform_u32(uint32_t v) { return __builtin_amdgcn_readfirstlane(v); }

__device__ __forceinline__ uint32_t brv(uint32_t x, uint32_t bits) { return __builtin_bitreverse32(x) >> (32 - bits); }

// Galois permutation of NTT slots (include/galois.cuh:98-113):
//   pi(i) = brv(((elt * brv(N + i, logN + 1)) >> 1) mod N, logN),
// with brv(N + i, logN + 1) = 2 brv(i, logN) + 1.
__device__ __forceinline__ uint32_t galois_perm(uint32_t elt, uint32_t i, uint32_t logN) {
    const uint64_t rev = 2ull * brv(i, logN) + 1;
    const uint32_t raw = (uint32_t)((elt * rev) >> 1) & ((1u << logN) - 1);
    return brv(raw, logN);
}

// Two adjacent residues moved as one 16-byte access, with the streaming hints
// of ld_stream / st_stream.
using u64x2 = unsigned long long __attribute__((ext_vector_type(2)));
__device__ __forceinline__ u64x2 ld_stream2(const uint64_t *p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u64x2 *>(p));
}
__device__ __forceinline__ void st_stream2(uint64_t *p, uint64_t x, uint64_t y) {
    u64x2 v;
    v.x = x;
    v.y = y;
    __builtin_nontemporal_store(v, reinterpret_cast<u64x2 *>(p));
}

// One residue of the degree-2 tensor product (a0 + a1 s)(b0 + b1 s) mod q
// (tensor_prod_2x2_rns_poly, src/polymath.cu:463-498): d0 = a0 b0,
// d1 = a0 b1 + a1 b0, d2 = a1 b1, all canonical.  FP64 policy (q < 2^50):
// |a b / q| < q < 2^50 keeps fl(a fl(b/q)) within 3/8 of the true quotient, so
// each product is within 0.875 q and a sum of two stays far below 2^53.
__device__ __forceinline__ void tensor_elem(const ArithF64 &ar, uint64_t a0, uint64_t a1, uint64_t b0, uint64_t b1,
                                            uint64_t &d0, uint64_t &d1, uint64_t &d2) {
    const double x0 = ar.load(a0), x1 = ar.load(a1), y0 = ar.load(b0), y1 = ar.load(b1);
    const double q0 = y0 * ar.qinv, q1 = y1 * ar.qinv;
    d0 = ar.store(ar.mulw(x0, y0, q0));
    d1 = ar.store(ar.mulw(x0, y1, q1) + ar.mulw(x1, y0, q0));
    d2 = ar.store(ar.mulw(x1, y1, q1));
}
// Integer policy: Barrett reduction of each 128-bit product or sum of two
// (r = floor(2^128 / q) as (lo, hi)).
__device__ __forceinline__ void tensor_elem(uint64_t q, ulonglong2 r, uint64_t a0, uint64_t a1, uint64_t b0,
                                            uint64_t b1, uint64_t &d0, uint64_t &d1, uint64_t &d2) {
    U128 m{0, 0};
    mac(m, a0, b1);
    mac(m, a1, b0);
    d0 = barrett128(U128{a0 * b0, mulhi64(a0, b0)}, q, r.x, r.y);
    d1 = barrett128(m, q, r.x, r.y);
    d2 = barrett128(U128{a1 * b1, mulhi64(a1, b1)}, q, r.x, r.y);
}

}  // namespace pfa
