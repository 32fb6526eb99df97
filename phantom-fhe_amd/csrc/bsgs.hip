// BSGS matrix-vector product support (src/bsgs.cu):
// * the giant-step accumulation of bsgs_apply_giants_with_babies
//   (mac_accumulate_kernel, src/bsgs.cu:51-96, used by build_partial,
//   :276-342) for every giant in one launch;
// * the batched expansion of level-independent plaintexts (signed
//   coefficients, light_pt_expand_per_tower_kernel, src/bsgs.cu:16-23);
// * native drivers of the baby-step chain (compute_bsgs_babies, :194-214) and
//   of the giant-step Horner loop with its rescale (:344-356), one C-ABI call
//   each, so a product costs two host calls instead of ~1100 launches from the
//   caller's language.
//
// Accumulation: out[g][k][j] = sum_{b < M} pt[g M + b][j] * baby[b][k][j]
// (mod q_j) for giant g, ciphertext poly k in {0, 1} and limb j.  The reference
// runs one launch per giant, reading all M babies each time.  Results are
// canonical residues, equal to the reference's per-step Barrett sums.
#include "internal.h"
#include "ntt_kernels.h"

namespace pfa {

namespace {

constexpr int kThreads = 256;

// Pointer list of the accumulation: a device table, or (no table) an
// arithmetic progression base + i * stride, which is how contiguous batches of
// plaintexts and outputs arrive; neither needs a host-to-device copy.
template <class P>
struct PtrList {
    P *const *table;
    P *base;
    uint64_t stride;  // elements
    // entry i (a wave-uniform index): table entries are read with scalar
    // loads, which do not queue behind the vector loads in flight
    __device__ __forceinline__ P *operator[](size_t i) const {
        return table ? reinterpret_cast<P *>(ld_const(reinterpret_cast<const uint64_t *>(table + i)))
                     : base + i * stride;
    }
};

// Residues per span of the tiled plaintext layout (and per accumulation work item).
constexpr uint32_t kSpan = 512;
constexpr int kPer = kSpan / kThreads;  // adjacent residues per thread (one 16-byte load)
static_assert(kPer == 2, "pair loads");

typedef uint64_t Pair __attribute__((ext_vector_type(2)));
typedef const __attribute__((address_space(1))) Pair *GlobalPair;  // pointers here are all device memory
__device__ __forceinline__ Pair ld_pair_stream(const uint64_t *p) {
    return __builtin_nontemporal_load((GlobalPair)p);
}
__device__ __forceinline__ Pair ld_pair(const uint64_t *p) { return *(GlobalPair)p; }
__device__ __forceinline__ void st_pair_stream(uint64_t *p, Pair v) {
    __builtin_nontemporal_store(v, (__attribute__((address_space(1))) Pair *)p);
}

// The tiled plaintext layout (pfa_bsgs_tile_plaintexts) of a set of D
// plaintexts: one region per limb j at byte offset off[j], holding span t of
// plaintext d at position (t D + d) kSpan.  A limb whose prime is below 2^40
// is packed: its region is D N 32-bit low words, then D N bytes of bits
// 32..39 (5 bytes per residue instead of 8); the accumulation is bound by
// reading this set, so packing cuts its time with its size.
constexpr uint32_t kMaxTiledLimbs = 64;
constexpr uint64_t kPackBound = 1ull << 40;
struct TiledLayout {
    uint64_t off[kMaxTiledLimbs];
    uint64_t packed;  // bit j: limb j is packed
    uint64_t bytes;   // total size
};

TiledLayout tiled_layout(const Ctx &c, uint32_t Ql, uint64_t D) {
    require(Ql <= kMaxTiledLimbs, "too many limbs for the tiled plaintext layout");
    TiledLayout t{};
    for (uint32_t j = 0; j < Ql; j++) {
        const bool pk = c.moduli[j] < kPackBound;
        t.off[j] = t.bytes;
        if (pk) t.packed |= 1ull << j;
        t.bytes += D * c.N * (pk ? 5 : 8);
    }
    return t;
}

struct MacArgs {
    PtrList<const uint64_t> pt;  // [G M] plaintexts, [Ql][N] each (NTT form), when tiled is null
    const uint8_t *tiled;        // or the same set in the tiled layout (pfa_bsgs_tile_plaintexts)
    TiledLayout lay;
    PtrList<uint64_t> out;       // [G] ciphertexts, [2][Ql][N] each
    PtrList<const uint64_t> babies;  // [M] ciphertexts, [2][Ql][N] each
    uint32_t M, G, Ql, N;
    uint32_t gb_begin, gb_end;  // giant blocks [gb_begin, gb_end) of kGB giants this launch covers
    __device__ __forceinline__ const uint64_t *baby(uint32_t b) const { return babies[b]; }
    // this thread's kPer residues of span `tile` of limb j of plaintext d
    __device__ __forceinline__ Pair span(uint32_t d, uint32_t j, uint32_t tile) const;
};

__device__ __forceinline__ Pair MacArgs::span(uint32_t d, uint32_t j, uint32_t tile) const {
    if (!tiled) return ld_pair_stream(pt[d] + (size_t)j * N + tile * kSpan + kPer * threadIdx.x);
    const size_t i = ((size_t)tile * ((size_t)G * M) + d) * kSpan + kPer * threadIdx.x;
    const uint8_t *r = tiled + lay.off[j];
    if (!((lay.packed >> j) & 1u)) return ld_pair_stream(reinterpret_cast<const uint64_t *>(r) + i);
    const uint64_t lo = __builtin_nontemporal_load(reinterpret_cast<const uint64_t *>(r) + i / 2);
    const uint32_t hi = __builtin_nontemporal_load(reinterpret_cast<const uint16_t *>(r + (size_t)G * M * N * 4) + i / 2);
    return Pair{(lo & 0xffffffffull) | ((uint64_t)(hi & 0xffu) << 32), (lo >> 32) | ((uint64_t)(hi >> 8) << 32)};
}

// giants per accumulation work item
constexpr uint32_t kGB = 8;

// Where an item's plaintext spans come from (uniform per item: a limb is
// packed or not, the set tiled or a pointer list).
enum SpanSrc { kSrcList = 0, kSrcTiled = 1, kSrcPacked = 2 };

// The kGB plaintext spans one baby step of an item multiplies (giants g0 ..
// g0 + kGB - 1; past the set's last giant, a repeat of the block's first,
// whose products are never stored).  All loads are issued before any value is
// used and none sits under a branch, so each wave keeps kGB loads in flight:
// with one load waited for at a time, an item reads 640 B per wave round trip
// and the accumulation ran at 2.8 TB/s.
template <int SRC>
__device__ __forceinline__ void load_spans(const MacArgs &a, uint32_t g0, uint32_t K, uint32_t b, uint32_t j,
                                           uint32_t tile, Pair (&xv)[kGB]) {
    if constexpr (SRC == kSrcList) {
#pragma unroll
        for (uint32_t k = 0; k < kGB; k++) xv[k] = a.span((g0 + (k < K ? k : 0)) * a.M + b, j, tile);
    } else {
        const size_t base = (size_t)tile * ((size_t)a.G * a.M) * kSpan + kPer * threadIdx.x;
        const uint8_t *r = a.tiled + a.lay.off[j];
        if constexpr (SRC == kSrcTiled) {
#pragma unroll
            for (uint32_t k = 0; k < kGB; k++) {
                const size_t d = (size_t)(g0 + (k < K ? k : 0)) * a.M + b;
                xv[k] = ld_pair_stream(reinterpret_cast<const uint64_t *>(r) + base + d * kSpan);
            }
        } else {
            const uint64_t *lo = reinterpret_cast<const uint64_t *>(r);
            const uint16_t *hi = reinterpret_cast<const uint16_t *>(r + (size_t)a.G * a.M * a.N * 4);
            uint64_t l[kGB];
            uint32_t h[kGB];
#pragma unroll
            for (uint32_t k = 0; k < kGB; k++) {
                const size_t i = base + (size_t)((g0 + (k < K ? k : 0)) * a.M + b) * kSpan;
                l[k] = __builtin_nontemporal_load(lo + i / 2);
                h[k] = __builtin_nontemporal_load(hi + i / 2);
            }
#pragma unroll
            for (uint32_t k = 0; k < kGB; k++)
                xv[k] = Pair{(l[k] & 0xffffffffull) | ((uint64_t)(h[k] & 0xffu) << 32),
                             (l[k] >> 32) | ((uint64_t)(h[k] >> 8) << 32)};
        }
    }
}

// One baby step's loads: the kGB plaintext spans and baby b's residues of both polys.
template <int SRC>
__device__ __forceinline__ void load_step(const MacArgs &a, uint32_t g0, uint32_t K, uint32_t b, uint32_t j,
                                          uint32_t tile, size_t off0, size_t off1, Pair (&xv)[kGB], Pair &c0,
                                          Pair &c1) {
    const uint64_t *c = a.baby(b);
    c0 = ld_pair(c + off0);
    c1 = ld_pair(c + off1);
    load_spans<SRC>(a, g0, K, b, j, tile, xv);
}

// A work item is (limb j, kSpan consecutive residues, block of up to kGB
// giants).  Baby b's residues are loaded once per item (kPer adjacent ones per
// thread and poly) and multiplied into every giant of the block, so the
// babies are read G / kGB times in all instead of G times.  Items of one
// (limb, span) carry the same workgroup index mod 8 and run on one XCD, which
// then holds that span of the babies in its L2.  The plaintexts are read once
// each: from a pointer list they arrive in 4 KiB runs of kGB M different
// plaintexts (4.0 TB/s measured, all of it compulsory traffic: the scattered
// rows, not the bytes, limit it); from the tiled layout an item's plaintext
// spans are one contiguous 2 MiB region.
// FP64 policy: each product is within 0.875 q (|x y / q| < q < 2^50), so four
// of them on top of a reduced sum stay below 4 q < 2^53; integer policy:
// 128-bit sums of full products, reduced every 8 babies (Barrett).
template <int SRC, bool F64>
__device__ __forceinline__ void mac_item(const MacArgs &a, uint32_t j, uint32_t tile, uint32_t g0, uint32_t K,
                                         uint64_t q, const ulonglong2 *ratio) {
    const size_t off0 = (size_t)j * a.N + tile * kSpan + kPer * threadIdx.x;
    const size_t off1 = off0 + (size_t)a.Ql * a.N;
    if constexpr (F64) {
        const ArithF64 ar(q);
        double acc0[kGB][kPer], acc1[kGB][kPer];
#pragma unroll
        for (uint32_t k = 0; k < kGB; k++)
#pragma unroll
            for (int e = 0; e < kPer; e++) acc0[k][e] = acc1[k][e] = 0.0;
        // baby step b: the kGB spans times baby b's residues of both polys
        auto step = [&](const Pair (&xv)[kGB], Pair c0, Pair c1, uint32_t b) {
            double y0[kPer], y1[kPer], y0q[kPer], y1q[kPer];
#pragma unroll
            for (int e = 0; e < kPer; e++) {
                y0[e] = ar.load(c0[e]);
                y1[e] = ar.load(c1[e]);
                y0q[e] = y0[e] * ar.qinv;
                y1q[e] = y1[e] * ar.qinv;
            }
#pragma unroll
            for (uint32_t k = 0; k < kGB; k++)
#pragma unroll
                for (int e = 0; e < kPer; e++) {
                    const double x = ar.load(xv[k][e]);
                    acc0[k][e] += ar.mulw(x, y0[e], y0q[e]);
                    acc1[k][e] += ar.mulw(x, y1[e], y1q[e]);
                }
            if ((b & 3u) == 3u) {
#pragma unroll
                for (uint32_t k = 0; k < kGB; k++)
#pragma unroll
                    for (int e = 0; e < kPer; e++) {
                        ar.reduce(acc0[k][e]);
                        ar.reduce(acc1[k][e]);
                    }
            }
        };
        // Two register sets: the next step's loads are requested before this
        // step's products, so they are in flight while it computes.  Indices
        // past the last step repeat it (no load under a branch).
        Pair xa[kGB], xb[kGB], a0, a1, b0, b1;
        load_step<SRC>(a, g0, K, 0, j, tile, off0, off1, xa, a0, a1);
        for (uint32_t b = 0; b < a.M; b += 2) {
            load_step<SRC>(a, g0, K, b + 1 < a.M ? b + 1 : b, j, tile, off0, off1, xb, b0, b1);
            __builtin_amdgcn_sched_barrier(0);
            step(xa, a0, a1, b);
            __builtin_amdgcn_sched_barrier(0);
            load_step<SRC>(a, g0, K, b + 2 < a.M ? b + 2 : a.M - 1, j, tile, off0, off1, xa, a0, a1);
            __builtin_amdgcn_sched_barrier(0);
            if (b + 1 < a.M) step(xb, b0, b1, b + 1);
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (uint32_t k = 0; k < kGB; k++) {
            if (k < K) {
                uint64_t *o = a.out[g0 + k];
                st_pair_stream(o + off0, Pair{ar.store(acc0[k][0]), ar.store(acc0[k][1])});
                st_pair_stream(o + off1, Pair{ar.store(acc1[k][0]), ar.store(acc1[k][1])});
            }
        }
    } else {
        // 128-bit sums of the full products (4 multiplies each), folded by one
        // Barrett reduction every 8 babies: with q < 2^62 a product is below
        // 2^124, so a folded value (< q) plus 8 products stays below 2^128.
        // The same residues as reducing every product.
        ulonglong2 r = ratio[j];
        r.x = wave_uniform(r.x);
        r.y = wave_uniform(r.y);
        U128 acc0[kGB][kPer], acc1[kGB][kPer];
#pragma unroll
        for (uint32_t k = 0; k < kGB; k++)
#pragma unroll
            for (int e = 0; e < kPer; e++) acc0[k][e] = acc1[k][e] = U128{0, 0};
        for (uint32_t b = 0; b < a.M; b++) {
            const uint64_t *c = a.baby(b);
            const Pair c0 = ld_pair(c + off0), c1 = ld_pair(c + off1);
            Pair xv[kGB];
            load_spans<SRC>(a, g0, K, b, j, tile, xv);
#pragma unroll
            for (uint32_t k = 0; k < kGB; k++)
#pragma unroll
                for (int e = 0; e < kPer; e++) {
                    mac(acc0[k][e], xv[k][e], c0[e]);
                    mac(acc1[k][e], xv[k][e], c1[e]);
                }
            if ((b & 7u) == 7u) {
#pragma unroll
                for (uint32_t k = 0; k < kGB; k++)
#pragma unroll
                    for (int e = 0; e < kPer; e++) {
                        acc0[k][e] = U128{barrett128(acc0[k][e], q, r.x, r.y), 0};
                        acc1[k][e] = U128{barrett128(acc1[k][e], q, r.x, r.y), 0};
                    }
            }
        }
#pragma unroll
        for (uint32_t k = 0; k < kGB; k++) {
            if (k < K) {
                uint64_t *o = a.out[g0 + k];
                st_pair_stream(o + off0, Pair{barrett128(acc0[k][0], q, r.x, r.y), barrett128(acc0[k][1], q, r.x, r.y)});
                st_pair_stream(o + off1, Pair{barrett128(acc1[k][0], q, r.x, r.y), barrett128(acc1[k][1], q, r.x, r.y)});
            }
        }
    }
}

__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 8)))
k_bsgs_mac(MacArgs a, const uint64_t *mod, const ulonglong2 *ratio) {
    const uint32_t T = a.N / kSpan;               // spans per limb
    const uint32_t GB = a.gb_end - a.gb_begin;    // giant blocks of this launch
    const uint32_t groups = a.Ql * T;
    const uint32_t total = grouped_total(groups, GB);
    for (uint32_t w = blockIdx.x; w < total; w += gridDim.x) {
        uint32_t grp, gb;
        if (!grouped_item(w, groups, GB, grp, gb)) continue;
        gb += a.gb_begin;
        const uint32_t j = grp / T, tile = grp % T;
        const uint64_t q = wave_uniform(mod[j]);
        const uint32_t g0 = gb * kGB;
        const uint32_t K = a.G - g0 < kGB ? a.G - g0 : kGB;  // giants in this block
        const bool f64 = q < kF64PrimeBound;
        if (!a.tiled) {
            if (f64)
                mac_item<kSrcList, true>(a, j, tile, g0, K, q, ratio);
            else
                mac_item<kSrcList, false>(a, j, tile, g0, K, q, ratio);
        } else if ((a.lay.packed >> j) & 1u) {
            if (f64)
                mac_item<kSrcPacked, true>(a, j, tile, g0, K, q, ratio);
            else
                mac_item<kSrcPacked, false>(a, j, tile, g0, K, q, ratio);
        } else {
            if (f64)
                mac_item<kSrcTiled, true>(a, j, tile, g0, K, q, ratio);
            else
                mac_item<kSrcTiled, false>(a, j, tile, g0, K, q, ratio);
        }
    }
}

// n signed coefficient polys [n][N] -> residues [n][L][N] of table rows start..start+L-1
__global__ void __launch_bounds__(kThreads)
k_expand_signed(const int64_t *in, uint64_t *out, const uint64_t *mod, uint32_t L, uint32_t start, uint32_t N) {
    const uint32_t l = blockIdx.y, p = blockIdx.z, n = blockIdx.x * kThreads + threadIdx.x;
    const uint64_t q = mod[start + l];
    const int64_t v = in[(size_t)p * N + n];
    uint64_t r;
    if (v >= 0) {
        r = (uint64_t)v % q;
    } else {
        r = (uint64_t)(-(v + 1)) % q;  // |v| - 1, no overflow at INT64_MIN
        r = q - 1 - r;
    }
    st_stream(out + ((size_t)p * L + l) * N + n, r);
}

// Plaintexts src[n][Ql][N] -> positions d0 .. d0+n-1 of a tiled set of D
// (TiledLayout): residue i of span t of limb j of plaintext d at position
// (t D + d) kSpan + i of limb j's region.  One workgroup per (span, limb,
// plaintext): a contiguous 4 KiB read, a contiguous 4 KiB (or 2.5 KiB) write.
__global__ void __launch_bounds__(kThreads)
k_bsgs_tile(const uint64_t *src, uint8_t *tiled, TiledLayout lay, uint32_t Ql, uint32_t N, uint32_t d0, uint32_t D) {
    const uint32_t t = blockIdx.x, j = blockIdx.y, p = blockIdx.z;
    const uint64_t *s = src + ((size_t)p * Ql + j) * N + (size_t)t * kSpan;
    const size_t pos = ((size_t)t * D + d0 + p) * kSpan;
    uint8_t *r = tiled + lay.off[j];
    if ((lay.packed >> j) & 1u) {
        uint32_t *lo = reinterpret_cast<uint32_t *>(r) + pos;
        uint8_t *hi = r + (size_t)D * N * 4 + pos;
#pragma unroll
        for (uint32_t i = threadIdx.x; i < kSpan; i += kThreads) {
            const uint64_t v = ld_stream(s + i);
            lo[i] = (uint32_t)v;
            hi[i] = (uint8_t)(v >> 32);
        }
        return;
    }
    uint64_t *o = reinterpret_cast<uint64_t *>(r) + pos;
#pragma unroll
    for (uint32_t i = threadIdx.x; i < kSpan; i += kThreads) st_stream(o + i, ld_stream(s + i));
}

// Both polys of B ciphertexts through the Galois permutation of NTT slots
// (apply_galois_ntt_permutation, src/galois.cu:11-18): ciphertext i of src
// (stride src_stride) -> ciphertext i of dst (contiguous [B][2][L][N]),
//   dst[i][k][l][n] = src[i][k][l][pi(n)]  (+ add0[l][n] for k = 0 when add0 is given, B = 1).
// With elts (a device table), ciphertext i uses its own element elts[i].
__global__ void __launch_bounds__(kThreads)
k_galois_ct(const uint64_t *src, uint64_t src_stride, uint64_t *dst, const uint64_t *add0, const uint64_t *mod,
            uint32_t elt, const uint32_t *elts, uint32_t L, uint32_t N, uint32_t logN) {
    const uint32_t l = blockIdx.y, k = blockIdx.z & 1u, i = blockIdx.z >> 1, n = blockIdx.x * kThreads + threadIdx.x;
    const size_t row = ((size_t)k * L + l) * N;
    const uint32_t e = elts ? elts[i] : elt;
    uint64_t v = src[i * src_stride + row + galois_perm(e, n, logN)];
    if (k == 0 && add0) v = add_mod(v, add0[(size_t)l * N + n], mod[l]);
    st_stream(dst + (size_t)i * 2 * L * N + row + n, v);
}

// out[i] = rotate(src[i]) for B ciphertexts with one key (+ add, B = 1): the
// Galois permutation of both polys, then the key switch of the permuted c1s
// whose ModDown epilogue adds the permuted c0 (and add[0]) to poly 0 and
// add[1] to poly 1 -- apply_galois_with_ksk (src/evaluate.cu:1607-1656),
// followed by add_inplace, with the same residues.  src[i] is at
// src + i src_stride, out is contiguous [B][2][Ql][N] and must not overlap
// src; add[1] may alias out's poly 1.
// With elts / keys (host arrays of B entries), ciphertext i is rotated by its
// own element with its own key (elt, key unused): the same residues as B
// single rotations.
void rotate_into(const Ctx &c, uint32_t chain, const uint64_t *src, uint64_t src_stride, uint32_t B, uint32_t elt,
                 const uint64_t *key, const uint64_t *add, uint64_t *out, hipStream_t s,
                 const uint32_t *elts = nullptr, const uint64_t *const *keys = nullptr) {
    const uint32_t Ql = c.size_Ql(chain), QlP = Ql + c.P;
    const uint64_t LN = (uint64_t)Ql * c.N;
    require(B >= 1 && B <= 32767 && (B == 1 || add == nullptr), "bad rotation batch");
    require((elts == nullptr) == (keys == nullptr), "per-rotation elements and keys go together");
    Scratch sc(c, s);
    uint32_t *elt_dev = nullptr;
    const uint64_t **key_dev = nullptr;
    if (elts) {
        void *dev[2];
        upload_parts(c, sc, s, {{elts, B * sizeof(uint32_t)}, {keys, B * sizeof(void *)}}, dev);
        elt_dev = (uint32_t *)dev[0];
        key_dev = (const uint64_t **)dev[1];
    }
    uint64_t *t = sc.alloc((size_t)B * 2 * LN);
    // up to N = 2^16 the permutation kernel also runs the first pass of the
    // key switch's INTT over the permuted c1 (mid), as the HMult tensor kernel does
    uint64_t *mid = nullptr;
    if (c.logN <= 16) {
        mid = sc.alloc((size_t)B * LN);
        galois_rows(c, chain, src, src_stride, B, elt, elt_dev, add, t, mid, s);
    } else {
        hipLaunchKernelGGL(k_galois_ct, dim3(c.N / kThreads, Ql, 2 * B), dim3(kThreads), 0, s, src, src_stride, t,
                           add, c.mod, elt, elt_dev, Ql, c.N, c.logN);
        PFA_HIP(hipGetLastError());
    }
    uint64_t *cx = sc.alloc((size_t)B * 2 * QlP * c.N);
    fused_modup_inner(c, chain, t + LN, key, cx, s, B, 2 * LN, (uint64_t)2 * QlP * c.N, nullptr, key_dev, mid);
    fused_moddown(c, chain, cx, 2 * B, out, t, add ? add + LN : nullptr, s, 2 * LN);
}

// Accumulation arguments: plaintexts from the pointer list pts or the tiled
// set, pointer tables (when a list is not an arithmetic progression) copied to
// workspace memory on stream s.
MacArgs mac_args(const Ctx &c, size_t chain_index, const uint64_t *const *pts, const uint64_t *tiled,
                 const uint64_t *const *babies, size_t M, size_t G, uint64_t *const *out, Scratch &sc,
                 hipStream_t s) {
    require(babies && out, "null argument");
    require(M >= 1 && G >= 1, "need at least one baby step and one giant step");
    require(M * G < (1u << 24), "too many plaintexts");
    if (chain_index < 1 || chain_index > c.Q) fail(PFA_ERR_INVALID_ARGUMENT, "chain index out of range");
    for (size_t i = 0; i < M; i++) require(babies[i] != nullptr, "null ciphertext pointer");
    for (size_t i = 0; i < G; i++) require(out[i] != nullptr, "null output pointer");
    MacArgs a{};
    a.M = (uint32_t)M;
    a.G = (uint32_t)G;
    a.Ql = c.size_Ql((uint32_t)chain_index);
    a.N = c.N;
    a.gb_begin = 0;
    a.gb_end = ((uint32_t)G + kGB - 1) / kGB;
    // a list whose addresses step by a constant multiple of 8 bytes goes as base + stride
    auto progression = [](const void *const *v, size_t n, uint64_t &stride) {
        const uintptr_t b0 = (uintptr_t)v[0];
        const intptr_t d = n > 1 ? (intptr_t)((uintptr_t)v[1] - b0) : 0;
        if (d < 0 || d % 8) return false;
        for (size_t i = 1; i < n; i++)
            if ((uintptr_t)v[i] != b0 + (uintptr_t)d * i) return false;
        stride = (uint64_t)d / 8;
        return true;
    };
    uint64_t st = 0;
    a.tiled = reinterpret_cast<const uint8_t *>(tiled);
    if (tiled) a.lay = tiled_layout(c, a.Ql, (uint64_t)M * G);
    // lists that are not arithmetic progressions go as tables, uploaded together
    const bool pt_tab = !tiled && !progression((const void *const *)pts, M * G, st);
    if (!tiled && !pt_tab) a.pt = PtrList<const uint64_t>{nullptr, pts[0], st};
    const bool out_tab = !progression((const void *const *)out, G, st);
    if (!out_tab) a.out = PtrList<uint64_t>{nullptr, out[0], st};
    const bool bab_tab = !progression((const void *const *)babies, M, st);
    if (!bab_tab) a.babies = PtrList<const uint64_t>{nullptr, babies[0], st};
    void *dev[3];
    upload_parts(c, sc, s,
                 {{pts, pt_tab ? M * G * sizeof(void *) : 0}, {out, out_tab ? G * sizeof(void *) : 0},
                  {babies, bab_tab ? M * sizeof(void *) : 0}},
                 dev);
    if (pt_tab) a.pt = PtrList<const uint64_t>{(const uint64_t *const *)dev[0], nullptr, 0};
    if (out_tab) a.out = PtrList<uint64_t>{(uint64_t *const *)dev[1], nullptr, 0};
    if (bab_tab) a.babies = PtrList<const uint64_t>{(const uint64_t *const *)dev[2], nullptr, 0};
    return a;
}

// one launch over giant blocks [a.gb_begin, a.gb_end), at most wpc workgroups per CU
void launch_mac(const Ctx &c, const MacArgs &a, uint32_t wpc, hipStream_t s) {
    const uint32_t total = grouped_total(a.Ql * (c.N / kSpan), a.gb_end - a.gb_begin);
    const uint32_t cap = (uint32_t)c.n_cu * wpc;
    hipLaunchKernelGGL(k_bsgs_mac, dim3(total < cap ? total : cap), dim3(kThreads), 0, s, a, c.mod, c.ratio);
    PFA_HIP(hipGetLastError());
}

uint32_t rotation_elt(const Ctx &c, int step) {
    uint32_t e = 0;
    if (pfa_galois_elt_from_step(step, c.N, &e) != PFA_OK) fail(PFA_ERR_INVALID_ARGUMENT, "bad rotation step");
    return e;
}

void check_key(const Ctx &c, uint32_t chain, const uint64_t *key, size_t dnum) {
    require(key != nullptr, "null Galois key");
    require(c.level(chain).beta <= dnum, "key has fewer digits than the ciphertext level needs");
}

}  // namespace

}  // namespace pfa

using namespace pfa;

extern "C" {

int pfa_bsgs_mac(const pfa_context *ctx, size_t chain_index, const uint64_t *const *pts,
                 const uint64_t *const *babies, size_t M, size_t G, uint64_t *const *out, void *stream) {
    return guarded([&] {
        require(pts != nullptr, "null argument");
        for (size_t i = 0; i < M * G; i++) require(pts[i] != nullptr, "null plaintext pointer");
        const Ctx &c = *ctx_of(ctx);
        const hipStream_t s = as_stream(stream);
        Scratch sc(c, s);
        // 4 resident workgroups per CU (119 VGPRs: 4 waves per SIMD)
        launch_mac(c, mac_args(c, chain_index, pts, nullptr, babies, M, G, out, sc, s), 4, s);
    });
}

int pfa_bsgs_mac_tiled(const pfa_context *ctx, size_t chain_index, const uint64_t *tiled,
                       const uint64_t *const *babies, size_t M, size_t G, uint64_t *const *out, void *stream) {
    return guarded([&] {
        require(tiled != nullptr, "null argument");
        const Ctx &c = *ctx_of(ctx);
        const hipStream_t s = as_stream(stream);
        Scratch sc(c, s);
        launch_mac(c, mac_args(c, chain_index, nullptr, tiled, babies, M, G, out, sc, s), 4, s);
    });
}

int pfa_bsgs_tile_plaintexts(const pfa_context *ctx, size_t chain_index, const uint64_t *src, size_t n,
                             uint64_t *tiled, size_t d0, size_t D, void *stream) {
    return guarded([&] {
        const Ctx &c = *ctx_of(ctx);
        require(src && tiled, "null argument");
        if (chain_index < 1 || chain_index > c.Q) fail(PFA_ERR_INVALID_ARGUMENT, "chain index out of range");
        require(n >= 1 && n <= 65535 && d0 + n <= D && D < (1u << 24), "plaintext range out of bounds");
        const uint32_t Ql = c.size_Ql((uint32_t)chain_index);
        const TiledLayout lay = tiled_layout(c, Ql, D);
        hipLaunchKernelGGL(k_bsgs_tile, dim3(c.N / kSpan, Ql, (uint32_t)n), dim3(kThreads), 0, as_stream(stream), src,
                           reinterpret_cast<uint8_t *>(tiled), lay, Ql, c.N, (uint32_t)d0, (uint32_t)D);
        PFA_HIP(hipGetLastError());
    });
}

int pfa_rotate_batch(const pfa_context *ctx, size_t chain_index, size_t count, const uint64_t *in,
                     const uint32_t *elts, const uint64_t *const *keys, size_t key_dnum, uint64_t *out,
                     void *stream) {
    return guarded([&] {
        const Ctx &c = *ctx_of(ctx);
        require(in && out && elts && keys, "null argument");
        require(count >= 1 && count <= 4096, "count out of range");
        if (chain_index < 1 || chain_index > c.Q) fail(PFA_ERR_INVALID_ARGUMENT, "chain index out of range");
        const uint32_t chain = (uint32_t)chain_index;
        const size_t ct_elems = (size_t)2 * c.size_Ql(chain) * c.N;
        require(out + count * ct_elems <= in || out >= in + count * ct_elems, "output overlaps the input");
        for (size_t i = 0; i < count; i++) {
            require((elts[i] & 1) && elts[i] < 2 * c.N, "bad Galois element");
            check_key(c, chain, keys[i], key_dnum);
        }
        if (count == 1)  // one element and key: no device tables to upload
            rotate_into(c, chain, in, ct_elems, 1, elts[0], keys[0], nullptr, out, as_stream(stream));
        else
            rotate_into(c, chain, in, ct_elems, (uint32_t)count, 0, nullptr, nullptr, out, as_stream(stream), elts,
                        keys);
    });
}

int pfa_bsgs_tiled_size(const pfa_context *ctx, size_t chain_index, size_t D, size_t *bytes) {
    return guarded([&] {
        const Ctx &c = *ctx_of(ctx);
        require(bytes != nullptr, "null argument");
        if (chain_index < 1 || chain_index > c.Q) fail(PFA_ERR_INVALID_ARGUMENT, "chain index out of range");
        require(D >= 1 && D < (1u << 24), "plaintext count out of range");
        *bytes = (size_t)tiled_layout(c, c.size_Ql((uint32_t)chain_index), D).bytes;
    });
}

int pfa_bsgs_babies(const pfa_context *ctx, size_t chain_index, const uint64_t *ct, size_t M,
                    const uint64_t *const *keys, size_t key_dnum, uint64_t *out, void *stream) {
    return guarded([&] {
        const Ctx &c = *ctx_of(ctx);
        require(ct && out && (M <= 1 || keys), "null argument");
        require(M >= 1 && M <= (size_t)c.N / 2, "baby step count out of range");
        if (chain_index < 1 || chain_index > c.Q) fail(PFA_ERR_INVALID_ARGUMENT, "chain index out of range");
        const uint32_t chain = (uint32_t)chain_index;
        std::vector<uint32_t> elts;
        for (size_t bit = 1, k = 0; bit < M; bit <<= 1, k++) {
            check_key(c, chain, keys[k], key_dnum);
            elts.push_back(rotation_elt(c, (int)bit));
        }
        const hipStream_t s = as_stream(stream);
        const uint64_t ct_elems = (uint64_t)2 * c.size_Ql(chain) * c.N;
        if (out != ct) PFA_HIP(hipMemcpyAsync(out, ct, ct_elems * 8, hipMemcpyDeviceToDevice, s));
        // babies[b] = rotate(babies[b - msb(b)], msb(b)): the babies with msb(b) = 2^k
        // are one rotation by 2^k of babies 0 .. 2^k - 1, run as one batch
        for (size_t bit = 1, k = 0; bit < M; bit <<= 1, k++) {
            const size_t B = std::min(bit, M - bit);
            for (size_t b0 = 0; b0 < B; b0 += 32767) {
                const size_t n = std::min<size_t>(32767, B - b0);
                rotate_into(c, chain, out + b0 * ct_elems, ct_elems, (uint32_t)n, elts[k], keys[k], nullptr,
                            out + (bit + b0) * ct_elems, s);
            }
        }
    });
}

int pfa_bsgs_giants(const pfa_context *ctx, size_t chain_index, uint64_t *partials, size_t G, int step,
                    const uint64_t *key, size_t key_dnum, uint64_t *out, void *stream) {
    return guarded([&] {
        const Ctx &c = *ctx_of(ctx);
        require(partials && out, "null argument");
        require(G >= 1, "need at least one giant step");
        if (chain_index < 1 || chain_index > c.Q) fail(PFA_ERR_INVALID_ARGUMENT, "chain index out of range");
        const uint32_t chain = (uint32_t)chain_index;
        require(c.size_Ql(chain) >= 2, "cannot rescale at the last level");
        const uint32_t elt = G > 1 ? rotation_elt(c, step) : 0;
        if (G > 1) check_key(c, chain, key, key_dnum);
        const hipStream_t s = as_stream(stream);
        const size_t ct_elems = (size_t)2 * c.size_Ql(chain) * c.N;
        // Horner from the last giant: partial[g] <- rotate(partial[g + 1], step) + partial[g]
        for (size_t g = G - 1; g-- > 0;) {
            uint64_t *pg = partials + g * ct_elems;
            rotate_into(c, chain, pg + ct_elems, 0, 1, elt, key, pg, pg, s);
        }
        fused_rescale(c, chain, partials, 2, out, s);
    });
}

int pfa_bsgs_apply_giants(const pfa_context *ctx, size_t chain_index, const uint64_t *tiled,
                          const uint64_t *const *babies, size_t M, size_t G, const uint64_t *key, size_t key_dnum,
                          uint64_t *out, void *stream) {
    return guarded([&] {
        const Ctx &c = *ctx_of(ctx);
        require(tiled && out, "null argument");
        if (chain_index < 1 || chain_index > c.Q) fail(PFA_ERR_INVALID_ARGUMENT, "chain index out of range");
        const uint32_t chain = (uint32_t)chain_index;
        require(c.size_Ql(chain) >= 2, "cannot rescale at the last level");
        require(M <= (size_t)INT32_MAX, "baby step count out of range");
        const uint32_t elt = G > 1 ? rotation_elt(c, (int)M) : 0;
        if (G > 1) check_key(c, chain, key, key_dnum);
        const hipStream_t s = as_stream(stream);
        const uint64_t ct_elems = (uint64_t)2 * c.size_Ql(chain) * c.N;
        Scratch sc(c, s);
        uint64_t *partials = G >= 1 ? sc.alloc((size_t)G * ct_elems) : nullptr;
        std::vector<uint64_t *> outs(G);
        for (size_t g = 0; g < G; g++) outs[g] = partials + g * ct_elems;
        // Every partial in one launch, then the Horner loop.  (Running the
        // accumulation in giant blocks on a second stream, overlapped with the
        // Horner steps, measured no faster: both halves slowed down ~2x.)
        launch_mac(c, mac_args(c, chain_index, nullptr, tiled, babies, M, G, outs.data(), sc, s), 4, s);
        // Horner from the last giant: partial[g] <- rotate(partial[g + 1], M) + partial[g]
        for (size_t g = G - 1; g-- > 0;) {
            uint64_t *pg = partials + g * ct_elems;
            rotate_into(c, chain, pg + ct_elems, 0, 1, elt, key, pg, pg, s);
        }
        fused_rescale(c, chain, partials, 2, out, s);
    });
}

int pfa_expand_signed(const pfa_context *ctx, const int64_t *in, size_t n, uint64_t *out, size_t L, size_t start,
                      void *stream) {
    return guarded([&] {
        const Ctx &c = *ctx_of(ctx);
        require(in && out, "null argument");
        require(n >= 1 && n <= 65535, "poly count out of range");
        require(L >= 1 && start + L <= c.QP, "limb range exceeds the context's primes");
        hipLaunchKernelGGL(k_expand_signed, dim3(c.N / kThreads, (uint32_t)L, (uint32_t)n), dim3(kThreads), 0,
                           as_stream(stream), in, out, c.mod, (uint32_t)L, (uint32_t)start, c.N);
        PFA_HIP(hipGetLastError());
    });
}

}  // extern "C"
