// Batched negacyclic NTT / INTT kernels for gfx950.
//
// Transform convention (the reference's, src/ntt/ntt_1d.cu:17-292 and
// src/host/ntt.cu:11-56): for a limb a of length N = 2^(S1+S2) over prime q,
//   forward : out[i] = sum_j a_j psi^((2 brv(i) + 1) j)   (bit-reversed order)
//   inverse : its exact inverse (N^-1 folded into the last stage).
// It is the radix-2 network "stage m = 1, 2, ..., N/2, block i uses tw[m+i]"
// with tw[brv(k)] = psi^k, executed here as two passes over HBM:
//
//   columns pass: N2 independent sub-transforms of size N1 = 2^S1 over
//                 k1 (element index k = k1 N2 + k2), twiddle tw[2^g + (k1 >> (S1-g))]
//   rows pass   : N1 sub-transforms of size N2 = 2^S2 over k2, twiddle
//                 tw[2^g (N1 + k1) + (k2 >> (S2-g))]
//
// Each sub-transform of size 2^S is held by 2^(S-LE) threads with E = 2^LE
// elements each (LE = ceil(S/2)); two register rounds of radix-E butterflies
// are joined by one transpose through LDS.  Global loads and stores are
// coalesced: 16 adjacent lanes always touch 16 adjacent uint64 (one 128 B line).
// The inverse runs the same network backwards with GS butterflies, rows first.
//
// Launch order is limb-major, poly-minor, tile-innermost: the tiles of one limb
// for every poly of the batch are adjacent in blockIdx and a multiple of 8
// apart, so they run on the same XCD close in time and share its L2 copy of
// the limb's twiddles.
#pragma once

#include "modarith.h"

namespace pfa {

// Which physical table row (prime) a batch limb uses; see NttBatch.
struct LimbMap {
    uint32_t start, split, split_base;
    __device__ __forceinline__ uint32_t row(uint32_t l) const {
        return l < split ? start + l : split_base + (l - split);
    }
};

struct NttBatch {
    const uint64_t *src;  // input  [M][..L..][N], poly stride sstride
    uint64_t *dst;        // output (may equal src), poly stride dstride
    uint64_t sstride, dstride;  // elements between consecutive polys (>= L * N)
    uint32_t M, L;
    LimbMap map;
    // limbs l in [ex_lo + m*ex_step, min(ex_lo + m*ex_step + ex_len, ex_cap)) of poly m
    // are left untouched (ModUp: a digit's own limbs are already in NTT form)
    uint32_t ex_lo, ex_step, ex_len, ex_cap;
    // optional per-limb scale applied after the inverse (pair table indexed by l)
    const ulonglong2 *scale;
    __device__ __forceinline__ bool excluded(uint32_t m, uint32_t l) const {
        uint32_t lo = ex_lo + m * ex_step;
        uint32_t hi = lo + ex_len;
        hi = hi < ex_cap ? hi : ex_cap;
        return l >= lo && l < hi;
    }
};

struct NttTables {
    const uint64_t *mod;         // [QP] primes
    const ulonglong2 *tw;        // [QP][N] forward pairs
    const ulonglong2 *itw;       // [QP][N] inverse pairs (itw[1] carries N^-1)
    const ulonglong2 *ninv;      // [QP] N^-1 pairs
    const ulonglong2 *small_fw;  // [QP][kSmall] psi^brv(j), j < kSmall
    const ulonglong2 *small_inv; // [QP][kSmall] psi^-brv(j), j < kSmall (no N^-1 fold)
    const ulonglong2 *rb_fw;     // [QP][S2][N1] tw[(N1 + k1) << g]: rows-pass stage bases
    const ulonglong2 *rb_inv;    // [QP][S2][N1] itw[(N1 + k1) << g]
};

constexpr int kSmall = 256;

// Twiddles whose index bits are disjoint factor: with brv additive on disjoint
// bits, tw[A + j] = psi^brv(A) psi^brv(j) = tw[A] * small[j] when the low bits
// of A that j occupies are zero.  In the rows pass every stage-g twiddle of row
// k1 is tw[((N1 + k1) << g) + j] with j < 2^g, so it is rb[g][k1] * small[j]:
// one entry of a compact per-row table (contiguous across the rows of a tile)
// times one of a 256-entry table, one modular product each (FP64 policy).  This
// replaces the full-size table, whose strided reads cost a cache line per use.

template <int S>
struct Sub {
    static constexpr int LE = (S + 1) / 2;
    static constexpr int E = 1 << LE;
    static constexpr int T = 1 << (S - LE);  // threads per sub-transform
};

// ---------------------------------------------------------------- rounds
// forward, stages g = 0 .. LE-1 on elements u = F + T e
template <class A, int S>
__device__ __forceinline__ void fwd_round_a(typename A::T (&x)[Sub<S>::E], const A &ar, const ulonglong2 *tw,
                                            uint32_t base) {
    constexpr int LE = Sub<S>::LE, E = Sub<S>::E;
#pragma unroll
    for (int g = 0; g < LE; g++) {
        const int d = E >> (g + 1);
#pragma unroll
        for (int e = 0; e < E; e++) {
            if (e & d) continue;
            ar.ct(x[e], x[e + d], tw[(base << g) + (e >> (LE - g))]);
        }
    }
}

// forward, stages g = LE .. S-1 on elements u = F' E + e
template <class A, int S>
__device__ __forceinline__ void fwd_round_b(typename A::T (&x)[Sub<S>::E], const A &ar, const ulonglong2 *tw,
                                            uint32_t base, uint32_t F) {
    constexpr int LE = Sub<S>::LE, E = Sub<S>::E;
#pragma unroll
    for (int g = LE; g < S; g++) {
        const int d = 1 << (S - 1 - g);
        const ulonglong2 *t = tw + (base << g) + (F << (LE - S + g));
#pragma unroll
        for (int e = 0; e < E; e++) {
            if (e & d) continue;
            ar.ct(x[e], x[e + d], t[e >> (S - g)]);
        }
    }
}

// inverse, stages g = S-1 .. LE on elements u = F' E + e
template <class A, int S>
__device__ __forceinline__ void inv_round_a(typename A::T (&x)[Sub<S>::E], const A &ar, const ulonglong2 *itw,
                                            uint32_t base, uint32_t F) {
    constexpr int LE = Sub<S>::LE, E = Sub<S>::E;
#pragma unroll
    for (int g = S - 1; g >= LE; g--) {
        const int d = 1 << (S - 1 - g);
        const ulonglong2 *t = itw + (base << g) + (F << (LE - S + g));
#pragma unroll
        for (int e = 0; e < E; e++) {
            if (e & d) continue;
            ar.gs(x[e], x[e + d], t[e >> (S - g)]);
        }
    }
}

// inverse, stages g = LE-1 .. 0 on elements u = F + T e.  With LAST the g = 0
// stage folds N^-1 into the sum half (the difference half gets it from itw[1]).
template <class A, int S, bool LAST>
__device__ __forceinline__ void inv_round_b(typename A::T (&x)[Sub<S>::E], const A &ar, const ulonglong2 *itw,
                                            uint32_t base, ulonglong2 ninv) {
    constexpr int LE = Sub<S>::LE, E = Sub<S>::E;
#pragma unroll
    for (int g = LE - 1; g >= 0; g--) {
        const int d = E >> (g + 1);
#pragma unroll
        for (int e = 0; e < E; e++) {
            if (e & d) continue;
            if (LAST && g == 0)
                ar.gs_last(x[e], x[e + d], itw[(base << g) + (e >> (LE - g))], ninv);
            else
                ar.gs(x[e], x[e + d], itw[(base << g) + (e >> (LE - g))]);
        }
    }
}

// Rows-pass rounds with derived twiddles (FP64 policy only).  rb points at this
// prime's [S][N1] base table, small at its kSmall table; k1 is the row.
template <int S, int N1>
__device__ __forceinline__ ulonglong2 rows_tw(const ArithF64 &ar, const ulonglong2 *rb, const ulonglong2 *small,
                                              uint32_t k1, int g, uint32_t j) {
    const ulonglong2 B = rb[g * N1 + k1];
    return j == 0 ? B : ar.twmul(B, small[j]);
}

// forward, stages g = 0 .. LE-1 on u = F + T e: j = e >> (LE - g)
template <int S, int N1>
__device__ __forceinline__ void fwd_round_a_derived(double (&x)[Sub<S>::E], const ArithF64 &ar,
                                                    const ulonglong2 *rb, const ulonglong2 *small, uint32_t k1) {
    constexpr int LE = Sub<S>::LE, E = Sub<S>::E;
#pragma unroll
    for (int g = 0; g < LE; g++) {
        const int d = E >> (g + 1);
        ulonglong2 w[1 << (LE - 1)];
#pragma unroll
        for (int i = 0; i < (1 << g); i++) w[i] = rows_tw<S, N1>(ar, rb, small, k1, g, i);
#pragma unroll
        for (int e = 0; e < E; e++) {
            if (e & d) continue;
            ar.ct(x[e], x[e + d], w[e >> (LE - g)]);
        }
    }
}

// forward, stages g = LE .. S-1 on u = F' E + e: j = (F' << (LE - S + g)) + (e >> (S - g))
template <int S, int N1>
__device__ __forceinline__ void fwd_round_b_derived(double (&x)[Sub<S>::E], const ArithF64 &ar,
                                                    const ulonglong2 *rb, const ulonglong2 *small, uint32_t k1,
                                                    uint32_t F) {
    constexpr int LE = Sub<S>::LE, E = Sub<S>::E;
#pragma unroll
    for (int g = LE; g < S; g++) {
        const int d = 1 << (S - 1 - g);
        const uint32_t jb = F << (LE - S + g);
        ulonglong2 w[1 << (LE - 1)];
#pragma unroll
        for (int i = 0; i < (1 << (g + LE - S)); i++) w[i] = rows_tw<S, N1>(ar, rb, small, k1, g, jb + i);
#pragma unroll
        for (int e = 0; e < E; e++) {
            if (e & d) continue;
            ar.ct(x[e], x[e + d], w[e >> (S - g)]);
        }
    }
}

// inverse, stages g = S-1 .. LE on u = F' E + e
template <int S, int N1>
__device__ __forceinline__ void inv_round_a_derived(double (&x)[Sub<S>::E], const ArithF64 &ar,
                                                    const ulonglong2 *rb, const ulonglong2 *small, uint32_t k1,
                                                    uint32_t F) {
    constexpr int LE = Sub<S>::LE, E = Sub<S>::E;
#pragma unroll
    for (int g = S - 1; g >= LE; g--) {
        const int d = 1 << (S - 1 - g);
        const uint32_t jb = F << (LE - S + g);
        ulonglong2 w[1 << (LE - 1)];
#pragma unroll
        for (int i = 0; i < (1 << (g + LE - S)); i++) w[i] = rows_tw<S, N1>(ar, rb, small, k1, g, jb + i);
#pragma unroll
        for (int e = 0; e < E; e++) {
            if (e & d) continue;
            ar.gs(x[e], x[e + d], w[e >> (S - g)]);
        }
    }
}

// inverse, stages g = LE-1 .. 0 on u = F + T e (rows pass: never the last stage)
template <int S, int N1>
__device__ __forceinline__ void inv_round_b_derived(double (&x)[Sub<S>::E], const ArithF64 &ar,
                                                    const ulonglong2 *rb, const ulonglong2 *small, uint32_t k1) {
    constexpr int LE = Sub<S>::LE, E = Sub<S>::E;
#pragma unroll
    for (int g = LE - 1; g >= 0; g--) {
        const int d = E >> (g + 1);
        ulonglong2 w[1 << (LE - 1)];
#pragma unroll
        for (int i = 0; i < (1 << g); i++) w[i] = rows_tw<S, N1>(ar, rb, small, k1, g, i);
#pragma unroll
        for (int e = 0; e < E; e++) {
            if (e & d) continue;
            ar.gs(x[e], x[e + d], w[e >> (LE - g)]);
        }
    }
}

// ---------------------------------------------------------------- tiling
// Columns pass: 16 adjacent columns per tile, T1 threads per column.
constexpr int kCols = 16;
// LDS row stride (in elements) for a [N1][kCols] column tile.
constexpr int kColStride = kCols + 1;

template <int S1, int S2>
struct Geo {
    static constexpr int N1 = 1 << S1, N2 = 1 << S2, LOGN = S1 + S2;
    static constexpr int N = 1 << LOGN;
    // columns pass
    static constexpr int COL_THREADS = kCols * Sub<S1>::T;
    static constexpr int COL_TILES = N2 / kCols;
    static constexpr int COL_LDS = N1 * kColStride;
    // rows pass: ROWS rows per tile, T2 threads per row (<= 256 threads,
    // <= 48 KiB of LDS)
    static constexpr int ROWS_BY_THREADS = 256 / Sub<S2>::T;
    static constexpr int ROWS_CAP = N2 >= 512 ? 8 : ROWS_BY_THREADS;
    static constexpr int ROWS = ROWS_CAP < N1 ? ROWS_CAP : N1;
    static constexpr int ROW_THREADS = ROWS * Sub<S2>::T;
    static constexpr int ROW_TILES = N1 / ROWS;
    // one pad slot every 16 elements: breaks the stride-E conflicts of round b
    static constexpr int ROW_PITCH = N2 + N2 / 16;
    static_assert(S1 <= 8, "column tile must fit in 64 KiB of LDS");
    static_assert(N2 >= kCols, "need at least 16 columns");
    static_assert((1 << (S2 - 1)) <= kSmall, "small twiddle table too short for the rows pass");
    static constexpr int ROW_LDS = ROWS * ROW_PITCH;
};

__device__ __forceinline__ int rpad(int k) { return k + (k >> 4); }

// Tiles are numbered limb-major, poly-minor, tile-innermost.  Each workgroup
// walks tiles blockIdx.x, blockIdx.x + gridDim.x, ... and prefetches the next
// tile's residues into registers while it transforms the current one, so HBM
// traffic overlaps the butterflies.
struct TileRef {
    uint32_t m, l, tile;
};

__device__ __forceinline__ TileRef decode_tile(const NttBatch &b, uint32_t tiles, uint32_t id) {
    TileRef r;
    r.tile = id % tiles;
    const uint32_t ml = id / tiles;
    r.m = ml % b.M;
    r.l = ml / b.M;
    return r;
}

// first tile id >= id (stepping by gridDim.x) that is not in an excluded limb
__device__ __forceinline__ uint32_t next_tile(const NttBatch &b, uint32_t tiles, uint32_t id, uint32_t total) {
    while (id < total) {
        const TileRef r = decode_tile(b, tiles, id);
        if (!b.excluded(r.m, r.l)) break;
        id += gridDim.x;
    }
    return id;
}

// ================================================================ forward
// Columns pass: src (canonical) -> dst (intermediate form).
template <int S1, int S2>
__device__ __forceinline__ const uint64_t *cols_src(const NttBatch &b, const TileRef &r, const uint64_t *base,
                                                    uint64_t stride) {
    using G = Geo<S1, S2>;
    return base + r.m * stride + (size_t)r.l * G::N + r.tile * kCols;
}

// Forward columns pass of one tile.  In: x[e] = element (F + T e) of column c
// of the tile, |x| <= q (any lazy representative).  Out: x[e] = element
// (F E + e) of the column in the intermediate form (lazy).
template <class A, int S1, int S2>
__device__ __forceinline__ void fwd_cols_core(typename A::T (&x)[Sub<S1>::E], const A &ar, const NttTables &t,
                                              uint32_t prow, typename A::T *lds) {
    using G = Geo<S1, S2>;
    using SB = Sub<S1>;
    const ulonglong2 *tw = t.tw + (size_t)prow * G::N;
    const uint32_t c = threadIdx.x % kCols, F = threadIdx.x / kCols;
    fwd_round_a<A, S1>(x, ar, tw, 1);
#pragma unroll
    for (int e = 0; e < SB::E; e++) {
        ar.reduce(x[e]);
        lds[(F + SB::T * e) * kColStride + c] = x[e];
    }
    __syncthreads();
#pragma unroll
    for (int e = 0; e < SB::E; e++) x[e] = lds[(F * SB::E + e) * kColStride + c];
    fwd_round_b<A, S1>(x, ar, tw, 1, F);
}

// store of fwd_cols_core's output into limb olimb (intermediate form)
template <class A, int S1, int S2>
__device__ __forceinline__ void fwd_cols_store(const typename A::T (&x)[Sub<S1>::E], const A &ar, uint32_t tile,
                                               uint64_t *olimb) {
    using G = Geo<S1, S2>;
    using SB = Sub<S1>;
    uint64_t *dst = olimb + tile * kCols;
    const uint32_t c = threadIdx.x % kCols, F = threadIdx.x / kCols;
#pragma unroll
    for (int e = 0; e < SB::E; e++) st_stream(&dst[(size_t)(F * SB::E + e) * G::N2 + c], ar.store_mid(x[e]));
}

template <class A, int S1, int S2>
__device__ __forceinline__ void fwd_cols_tile(const uint64_t (&raw)[Sub<S1>::E], const NttBatch &b,
                                              const NttTables &t, const TileRef &r, uint32_t prow, uint64_t q,
                                              typename A::T *lds, uint64_t *olimb) {
    using SB = Sub<S1>;
    using T = typename A::T;
    const A ar(q);
    T x[SB::E];
#pragma unroll
    for (int e = 0; e < SB::E; e++) x[e] = ar.load(raw[e]);
    fwd_cols_core<A, S1, S2>(x, ar, t, prow, lds);
    fwd_cols_store<A, S1, S2>(x, ar, r.tile, olimb);
}

template <int S1, int S2>
__global__ void __launch_bounds__((Geo<S1, S2>::COL_THREADS)) ntt_fwd_cols(NttBatch b, NttTables t) {
    using G = Geo<S1, S2>;
    using SB = Sub<S1>;
    __shared__ double lds[G::COL_LDS];
    const uint32_t total = b.M * b.L * G::COL_TILES;
    const uint32_t c = threadIdx.x % kCols, F = threadIdx.x / kCols;
    uint32_t cur = next_tile(b, G::COL_TILES, blockIdx.x, total);
    uint64_t raw[SB::E];
    if (cur < total) {
        const uint64_t *s = cols_src<S1, S2>(b, decode_tile(b, G::COL_TILES, cur), b.src, b.sstride);
#pragma unroll
        for (int e = 0; e < SB::E; e++) raw[e] = ld_stream(&s[(size_t)(F + SB::T * e) * G::N2 + c]);
    }
    while (cur < total) {
        const uint32_t nxt = next_tile(b, G::COL_TILES, cur + gridDim.x, total);
        const TileRef r = decode_tile(b, G::COL_TILES, cur);
        uint64_t nraw[SB::E];
        if (nxt < total) {
            const uint64_t *s = cols_src<S1, S2>(b, decode_tile(b, G::COL_TILES, nxt), b.src, b.sstride);
#pragma unroll
            for (int e = 0; e < SB::E; e++) nraw[e] = ld_stream(&s[(size_t)(F + SB::T * e) * G::N2 + c]);
        }
        const uint32_t prow = b.map.row(r.l);
        const uint64_t q = t.mod[prow];
        if (q < kF64PrimeBound)
            fwd_cols_tile<ArithF64, S1, S2>(raw, b, t, r, prow, q, lds, b.dst + r.m * b.dstride + (size_t)r.l * G::N);
        else
            fwd_cols_tile<ArithInt, S1, S2>(raw, b, t, r, prow, q, reinterpret_cast<uint64_t *>(lds), b.dst + r.m * b.dstride + (size_t)r.l * G::N);
#pragma unroll
        for (int e = 0; e < SB::E; e++) raw[e] = nraw[e];
        cur = nxt;
        __syncthreads();
    }
}

// Rows pass: dst (intermediate) -> dst (canonical).
// Forward rows pass of one tile row k1.  In: x[e] = element (F + T e) of the
// row in the intermediate form.  Out: x[e] = element (F + T e) of the
// transformed row (lazy; the final LDS transpose makes stores coalesced).
// The caller separates consecutive calls on the same LDS with a barrier.
template <class A, int S1, int S2>
__device__ __forceinline__ void fwd_rows_core(typename A::T (&x)[Sub<S2>::E], const A &ar, const NttTables &t,
                                              uint32_t prow, uint32_t k1, typename A::T *lr) {
    using G = Geo<S1, S2>;
    using SB = Sub<S2>;
    const ulonglong2 *tw = t.tw + (size_t)prow * G::N;
    const uint32_t F = threadIdx.x % SB::T;
    if constexpr (A::kF64)
        fwd_round_a_derived<S2, G::N1>(x, ar, t.rb_fw + (size_t)prow * S2 * G::N1, t.small_fw + (size_t)prow * kSmall, k1);
    else
        fwd_round_a<A, S2>(x, ar, tw, G::N1 + k1);
#pragma unroll
    for (int e = 0; e < SB::E; e++) {
        ar.reduce(x[e]);
        lr[rpad(F + SB::T * e)] = x[e];
    }
    __syncthreads();
#pragma unroll
    for (int e = 0; e < SB::E; e++) x[e] = lr[rpad(F * SB::E + e)];
    if constexpr (A::kF64)
        fwd_round_b_derived<S2, G::N1>(x, ar, t.rb_fw + (size_t)prow * S2 * G::N1, t.small_fw + (size_t)prow * kSmall, k1, F);
    else
        fwd_round_b<A, S2>(x, ar, tw, G::N1 + k1, F);
    __syncthreads();
#pragma unroll
    for (int e = 0; e < SB::E; e++) lr[rpad(F * SB::E + e)] = x[e];
    __syncthreads();
#pragma unroll
    for (int e = 0; e < SB::E; e++) x[e] = lr[rpad(F + SB::T * e)];
}

template <class A, int S1, int S2>
__device__ __forceinline__ void fwd_rows_tile(const uint64_t (&raw)[Sub<S2>::E], const NttBatch &b,
                                              const NttTables &t, const TileRef &r, uint32_t prow, uint64_t q,
                                              typename A::T *lds, uint64_t *olimb) {
    using G = Geo<S1, S2>;
    using SB = Sub<S2>;
    using T = typename A::T;
    const A ar(q);
    const uint32_t F = threadIdx.x % SB::T, rr = threadIdx.x / SB::T;
    const uint32_t k1 = r.tile * G::ROWS + rr;
    uint64_t *rowp = olimb + (size_t)k1 * G::N2;
    T x[SB::E];
#pragma unroll
    for (int e = 0; e < SB::E; e++) x[e] = ar.load_mid(raw[e]);
    fwd_rows_core<A, S1, S2>(x, ar, t, prow, k1, lds + rr * G::ROW_PITCH);
#pragma unroll
    for (int e = 0; e < SB::E; e++) st_stream(&rowp[F + SB::T * e], ar.store(x[e]));
}

template <int S1, int S2>
__device__ __forceinline__ const uint64_t *rows_ptr(const NttBatch &b, const TileRef &r, const uint64_t *base,
                                                    uint64_t stride) {
    using G = Geo<S1, S2>;
    const uint32_t rr = threadIdx.x / Sub<S2>::T;
    return base + r.m * stride + (size_t)r.l * G::N + (size_t)(r.tile * G::ROWS + rr) * G::N2;
}

template <int S1, int S2>
__global__ void __launch_bounds__((Geo<S1, S2>::ROW_THREADS)) ntt_fwd_rows(NttBatch b, NttTables t) {
    using G = Geo<S1, S2>;
    using SB = Sub<S2>;
    __shared__ double lds[G::ROW_LDS];
    const uint32_t total = b.M * b.L * G::ROW_TILES;
    const uint32_t F = threadIdx.x % SB::T;
    uint32_t cur = next_tile(b, G::ROW_TILES, blockIdx.x, total);
    uint64_t raw[SB::E];
    if (cur < total) {
        const uint64_t *s = rows_ptr<S1, S2>(b, decode_tile(b, G::ROW_TILES, cur), b.src, b.sstride);
#pragma unroll
        for (int e = 0; e < SB::E; e++) raw[e] = ld_stream(&s[F + SB::T * e]);
    }
    while (cur < total) {
        const uint32_t nxt = next_tile(b, G::ROW_TILES, cur + gridDim.x, total);
        const TileRef r = decode_tile(b, G::ROW_TILES, cur);
        uint64_t nraw[SB::E];
        if (nxt < total) {
            const uint64_t *s = rows_ptr<S1, S2>(b, decode_tile(b, G::ROW_TILES, nxt), b.src, b.sstride);
#pragma unroll
            for (int e = 0; e < SB::E; e++) nraw[e] = ld_stream(&s[F + SB::T * e]);
        }
        const uint32_t prow = b.map.row(r.l);
        const uint64_t q = t.mod[prow];
        if (q < kF64PrimeBound)
            fwd_rows_tile<ArithF64, S1, S2>(raw, b, t, r, prow, q, lds, b.dst + r.m * b.dstride + (size_t)r.l * G::N);
        else
            fwd_rows_tile<ArithInt, S1, S2>(raw, b, t, r, prow, q, reinterpret_cast<uint64_t *>(lds), b.dst + r.m * b.dstride + (size_t)r.l * G::N);
#pragma unroll
        for (int e = 0; e < SB::E; e++) raw[e] = nraw[e];
        cur = nxt;
        __syncthreads();
    }
}

// ================================================================ inverse
// Rows pass first: src (canonical) -> dst (intermediate).
template <class A, int S1, int S2>
__device__ __forceinline__ void inv_rows_tile(const uint64_t (&raw)[Sub<S2>::E], const NttBatch &b,
                                              const NttTables &t, const TileRef &r, uint32_t prow, uint64_t q,
                                              typename A::T *lds, uint64_t *olimb) {
    using G = Geo<S1, S2>;
    using SB = Sub<S2>;
    using T = typename A::T;
    const A ar(q);
    const ulonglong2 *itw = t.itw + (size_t)prow * G::N;
    const uint32_t F = threadIdx.x % SB::T, rr = threadIdx.x / SB::T;
    const uint32_t k1 = r.tile * G::ROWS + rr;
    uint64_t *drow = olimb + (size_t)k1 * G::N2;
    T *lr = lds + rr * G::ROW_PITCH;
    T x[SB::E];
#pragma unroll
    for (int e = 0; e < SB::E; e++) lr[rpad(F + SB::T * e)] = ar.load(raw[e]);
    __syncthreads();
#pragma unroll
    for (int e = 0; e < SB::E; e++) x[e] = lr[rpad(F * SB::E + e)];
    if constexpr (A::kF64)
        inv_round_a_derived<S2, G::N1>(x, ar, t.rb_inv + (size_t)prow * S2 * G::N1, t.small_inv + (size_t)prow * kSmall, k1, F);
    else
        inv_round_a<A, S2>(x, ar, itw, G::N1 + k1, F);
    __syncthreads();
#pragma unroll
    for (int e = 0; e < SB::E; e++) lr[rpad(F * SB::E + e)] = x[e];
    __syncthreads();
#pragma unroll
    for (int e = 0; e < SB::E; e++) x[e] = lr[rpad(F + SB::T * e)];
    if constexpr (A::kF64)
        inv_round_b_derived<S2, G::N1>(x, ar, t.rb_inv + (size_t)prow * S2 * G::N1, t.small_inv + (size_t)prow * kSmall, k1);
    else
        inv_round_b<A, S2, false>(x, ar, itw, G::N1 + k1, ulonglong2{0, 0});
#pragma unroll
    for (int e = 0; e < SB::E; e++) st_stream(&drow[F + SB::T * e], ar.store_mid(x[e]));
}

template <int S1, int S2>
__global__ void __launch_bounds__((Geo<S1, S2>::ROW_THREADS)) ntt_inv_rows(NttBatch b, NttTables t) {
    using G = Geo<S1, S2>;
    using SB = Sub<S2>;
    __shared__ double lds[G::ROW_LDS];
    const uint32_t total = b.M * b.L * G::ROW_TILES;
    const uint32_t F = threadIdx.x % SB::T;
    uint32_t cur = next_tile(b, G::ROW_TILES, blockIdx.x, total);
    uint64_t raw[SB::E];
    if (cur < total) {
        const uint64_t *s = rows_ptr<S1, S2>(b, decode_tile(b, G::ROW_TILES, cur), b.src, b.sstride);
#pragma unroll
        for (int e = 0; e < SB::E; e++) raw[e] = ld_stream(&s[F + SB::T * e]);
    }
    while (cur < total) {
        const uint32_t nxt = next_tile(b, G::ROW_TILES, cur + gridDim.x, total);
        const TileRef r = decode_tile(b, G::ROW_TILES, cur);
        uint64_t nraw[SB::E];
        if (nxt < total) {
            const uint64_t *s = rows_ptr<S1, S2>(b, decode_tile(b, G::ROW_TILES, nxt), b.src, b.sstride);
#pragma unroll
            for (int e = 0; e < SB::E; e++) nraw[e] = ld_stream(&s[F + SB::T * e]);
        }
        const uint32_t prow = b.map.row(r.l);
        const uint64_t q = t.mod[prow];
        if (q < kF64PrimeBound)
            inv_rows_tile<ArithF64, S1, S2>(raw, b, t, r, prow, q, lds, b.dst + r.m * b.dstride + (size_t)r.l * G::N);
        else
            inv_rows_tile<ArithInt, S1, S2>(raw, b, t, r, prow, q, reinterpret_cast<uint64_t *>(lds), b.dst + r.m * b.dstride + (size_t)r.l * G::N);
#pragma unroll
        for (int e = 0; e < SB::E; e++) raw[e] = nraw[e];
        cur = nxt;
        __syncthreads();
    }
}

// Columns pass: dst (intermediate) -> dst (canonical), N^-1 and optional scale.
template <class A, int S1, int S2>
__device__ __forceinline__ void inv_cols_tile(const uint64_t (&raw)[Sub<S1>::E], const NttBatch &b,
                                              const NttTables &t, const TileRef &r, uint32_t prow, uint64_t q,
                                              typename A::T *lds, uint64_t *olimb) {
    using G = Geo<S1, S2>;
    using SB = Sub<S1>;
    using T = typename A::T;
    const A ar(q);
    const ulonglong2 *itw = t.itw + (size_t)prow * G::N;
    uint64_t *data = olimb + r.tile * kCols;
    const uint32_t c = threadIdx.x % kCols, F = threadIdx.x / kCols;
    T x[SB::E];
#pragma unroll
    for (int e = 0; e < SB::E; e++) x[e] = ar.load_mid(raw[e]);
    inv_round_a<A, S1>(x, ar, itw, 1, F);
#pragma unroll
    for (int e = 0; e < SB::E; e++) lds[(F * SB::E + e) * kColStride + c] = x[e];
    __syncthreads();
#pragma unroll
    for (int e = 0; e < SB::E; e++) x[e] = lds[(F + SB::T * e) * kColStride + c];
    inv_round_b<A, S1, true>(x, ar, itw, 1, t.ninv[prow]);
    if (b.scale) {
        const ulonglong2 s = b.scale[r.l];
#pragma unroll
        for (int e = 0; e < SB::E; e++) ar.mul(x[e], s);
    }
#pragma unroll
    for (int e = 0; e < SB::E; e++) st_stream(&data[(size_t)(F + SB::T * e) * G::N2 + c], ar.store(x[e]));
}

template <int S1, int S2>
__global__ void __launch_bounds__((Geo<S1, S2>::COL_THREADS)) ntt_inv_cols(NttBatch b, NttTables t) {
    using G = Geo<S1, S2>;
    using SB = Sub<S1>;
    __shared__ double lds[G::COL_LDS];
    const uint32_t total = b.M * b.L * G::COL_TILES;
    const uint32_t c = threadIdx.x % kCols, F = threadIdx.x / kCols;
    uint32_t cur = next_tile(b, G::COL_TILES, blockIdx.x, total);
    uint64_t raw[SB::E];
    if (cur < total) {
        const uint64_t *s = cols_src<S1, S2>(b, decode_tile(b, G::COL_TILES, cur), b.src, b.sstride);
#pragma unroll
        for (int e = 0; e < SB::E; e++) raw[e] = ld_stream(&s[(size_t)(F * SB::E + e) * G::N2 + c]);
    }
    while (cur < total) {
        const uint32_t nxt = next_tile(b, G::COL_TILES, cur + gridDim.x, total);
        const TileRef r = decode_tile(b, G::COL_TILES, cur);
        uint64_t nraw[SB::E];
        if (nxt < total) {
            const uint64_t *s = cols_src<S1, S2>(b, decode_tile(b, G::COL_TILES, nxt), b.src, b.sstride);
#pragma unroll
            for (int e = 0; e < SB::E; e++) nraw[e] = ld_stream(&s[(size_t)(F * SB::E + e) * G::N2 + c]);
        }
        const uint32_t prow = b.map.row(r.l);
        const uint64_t q = t.mod[prow];
        if (q < kF64PrimeBound)
            inv_cols_tile<ArithF64, S1, S2>(raw, b, t, r, prow, q, lds, b.dst + r.m * b.dstride + (size_t)r.l * G::N);
        else
            inv_cols_tile<ArithInt, S1, S2>(raw, b, t, r, prow, q, reinterpret_cast<uint64_t *>(lds), b.dst + r.m * b.dstride + (size_t)r.l * G::N);
#pragma unroll
        for (int e = 0; e < SB::E; e++) raw[e] = nraw[e];
        cur = nxt;
        __syncthreads();
    }
}

}  // namespace pfa

namespace pfa {

// ================================================================ fused
// One launch runs both passes of every limb, with the intermediate kept in
// the L2 of one XCD:
//   * every workgroup reads its XCD id from the hardware register and takes
//     work only from that XCD's queue; limb-job j belongs to XCD j mod 8;
//   * a job is P1 tiles (first pass) then P2 tiles (second pass); the queue of
//     an XCD is ordered P1(0), P1(1), P2(0), P1(2), P2(1), ..., P2(n-1), so a P2
//     tile only ever waits for P1 tiles already taken by running workgroups
//     (no deadlock, whatever the residency), and waits are rare;
//   * P1 tiles store the intermediate into a per-job scratch limb (written
//     through to the XCD's L2), wait for the stores' acknowledgement, then bump
//     the job's counter (device-scope atomic); P2 tiles poll the counter and
//     read the scratch with plain loads from the shared L2.  No CU has
//     read a scratch line before within the launch (one limb per job), so no
//     L1 holds a stale copy, and the lines come from the shared L2.
// HBM sees the input read once, the output written once, plus the write-back
// of the dead scratch lines.  Every wait is bounded; on expiry a flag is raised
// and the kernel still terminates.
struct FusedCtl {
    uint32_t *queue;    // [8] per-XCD item counters, zero at launch
    uint32_t *done;     // [jobs] finished P1 tiles per job, zero at launch
    uint32_t *flags;    // [1] bit 0: a wait expired
    uint64_t *scratch;  // [jobs][N] intermediate, written by P1, read by P2
};

constexpr uint32_t kXcds = 8;
constexpr uint32_t kSpinLimit = 1u << 18;

__device__ __forceinline__ uint32_t xcc_id() {
    uint32_t v;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
    return v & (kXcds - 1);
}

struct FusedItem {
    uint32_t phase, k, tile;
};

// Queue order of one XCD with lag D (nx jobs, B tiles per phase of a job):
//   P1(0) .. P1(D-1), then P1(D), P2(0), P1(D+1), P2(1), ..., then the last P2s.
// P2(k) is taken about 2 D B items after P1(k) started, when its tiles are done.
__device__ __forceinline__ FusedItem fused_item(uint32_t it, uint32_t nx, uint32_t B, uint32_t D) {
    const uint32_t s = it / B, tile = it % B;
    const uint32_t d = nx < D ? nx : D;
    if (s < d) return FusedItem{1, s, tile};
    const uint32_t u = s - d, np = nx > D ? nx - D : 0;
    if (u < 2 * np) return (u & 1) ? FusedItem{2, u / 2, tile} : FusedItem{1, u / 2 + D, tile};
    return FusedItem{2, np + (u - 2 * np), tile};
}

// Queue and counters use device-scope atomics: on gfx950 workgroup-scope
// atomics are not coherent between CUs, so they cannot coordinate workgroups.
__device__ __forceinline__ uint32_t fused_take(uint32_t *queue, uint32_t xcc, uint32_t *s_slot) {
    if (threadIdx.x == 0)
        *s_slot = __hip_atomic_fetch_add(queue + xcc, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    const uint32_t it = *s_slot;
    __syncthreads();
    return it;
}

// P1 side: all of this workgroup's stores are acknowledged by L2, then count the tile.
__device__ __forceinline__ void fused_publish(uint32_t *done) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) __hip_atomic_fetch_add(done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// P2 side: wait until all `need` P1 tiles of the job are published.
__device__ __forceinline__ void fused_wait(uint32_t *done, uint32_t need, uint32_t *flags) {
    if (threadIdx.x == 0) {
        uint32_t spins = 0;
        while (__hip_atomic_load(done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < need) {
            __builtin_amdgcn_s_sleep(8);
            if (++spins > kSpinLimit) {
                __hip_atomic_fetch_or(flags, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
        }
    }
    __syncthreads();
}

template <int S1, int S2>
struct FusedGeo {
    using G = Geo<S1, S2>;
    static constexpr bool OK = G::COL_THREADS == 256 && G::ROW_THREADS == 256 && G::COL_LDS == G::ROW_LDS &&
                               G::COL_TILES == G::ROW_TILES;
    static constexpr int THREADS = 256;
    static constexpr int LDS = G::COL_LDS;
};

template <int S1, int S2>
__global__ void __launch_bounds__(256) ntt_fwd_fused(NttBatch b, NttTables t, FusedCtl ctl, uint32_t lag) {
    using G = Geo<S1, S2>;
    using S1B = Sub<S1>;
    using S2B = Sub<S2>;
    static_assert(FusedGeo<S1, S2>::OK, "fused NTT needs matching 256-thread passes");
    __shared__ double lds[FusedGeo<S1, S2>::LDS];
    __shared__ uint32_t s_slot;
    const uint32_t xcc = xcc_id();
    const uint32_t jobs = b.M * b.L;
    const uint32_t nx = jobs > xcc ? (jobs - xcc + kXcds - 1) / kXcds : 0;
    const uint32_t n1 = G::COL_TILES, n2 = G::ROW_TILES, total = nx * (n1 + n2);
    for (;;) {
        const uint32_t it = fused_take(ctl.queue, xcc, &s_slot);
        if (it >= total) break;
        const FusedItem f = fused_item(it, nx, n1, lag);
        const uint32_t job = xcc + kXcds * f.k;
        const TileRef r{job % b.M, job / b.M, f.tile};
        const bool skip = b.excluded(r.m, r.l);
        const uint32_t prow = b.map.row(r.l);
        const uint64_t q = t.mod[prow];
        if (f.phase == 1) {
            if (!skip) {
                const uint32_t c = threadIdx.x % kCols, F = threadIdx.x / kCols;
                const uint64_t *s = cols_src<S1, S2>(b, r, b.src, b.sstride);
                uint64_t raw[S1B::E];
#pragma unroll
                for (int e = 0; e < S1B::E; e++) raw[e] = ld_stream(&s[(size_t)(F + S1B::T * e) * G::N2 + c]);
                if (q < kF64PrimeBound)
                    fwd_cols_tile<ArithF64, S1, S2>(raw, b, t, r, prow, q, lds, ctl.scratch + (size_t)job * G::N);
                else
                    fwd_cols_tile<ArithInt, S1, S2>(raw, b, t, r, prow, q, reinterpret_cast<uint64_t *>(lds), ctl.scratch + (size_t)job * G::N);
            }
            fused_publish(ctl.done + job);
        } else if (!skip) {
            fused_wait(ctl.done + job, n1, ctl.flags);
            const uint32_t F = threadIdx.x % S2B::T, rr = threadIdx.x / S2B::T;
            const uint64_t *srow = ctl.scratch + (size_t)job * G::N + (size_t)(r.tile * G::ROWS + rr) * G::N2;
            uint64_t raw[S2B::E];
#pragma unroll
            for (int e = 0; e < S2B::E; e++) raw[e] = srow[F + S2B::T * e];
            if (q < kF64PrimeBound)
                fwd_rows_tile<ArithF64, S1, S2>(raw, b, t, r, prow, q, lds, b.dst + r.m * b.dstride + (size_t)r.l * G::N);
            else
                fwd_rows_tile<ArithInt, S1, S2>(raw, b, t, r, prow, q, reinterpret_cast<uint64_t *>(lds), b.dst + r.m * b.dstride + (size_t)r.l * G::N);
        }
        __syncthreads();
    }
}

template <int S1, int S2>
__global__ void __launch_bounds__(256) ntt_inv_fused(NttBatch b, NttTables t, FusedCtl ctl, uint32_t lag) {
    using G = Geo<S1, S2>;
    using S1B = Sub<S1>;
    using S2B = Sub<S2>;
    static_assert(FusedGeo<S1, S2>::OK, "fused NTT needs matching 256-thread passes");
    __shared__ double lds[FusedGeo<S1, S2>::LDS];
    __shared__ uint32_t s_slot;
    const uint32_t xcc = xcc_id();
    const uint32_t jobs = b.M * b.L;
    const uint32_t nx = jobs > xcc ? (jobs - xcc + kXcds - 1) / kXcds : 0;
    const uint32_t n1 = G::ROW_TILES, n2 = G::COL_TILES, total = nx * (n1 + n2);
    for (;;) {
        const uint32_t it = fused_take(ctl.queue, xcc, &s_slot);
        if (it >= total) break;
        const FusedItem f = fused_item(it, nx, n1, lag);
        const uint32_t job = xcc + kXcds * f.k;
        const TileRef r{job % b.M, job / b.M, f.tile};
        const bool skip = b.excluded(r.m, r.l);
        const uint32_t prow = b.map.row(r.l);
        const uint64_t q = t.mod[prow];
        if (f.phase == 1) {
            if (!skip) {
                const uint32_t F = threadIdx.x % S2B::T;
                const uint64_t *s = rows_ptr<S1, S2>(b, r, b.src, b.sstride);
                uint64_t raw[S2B::E];
#pragma unroll
                for (int e = 0; e < S2B::E; e++) raw[e] = ld_stream(&s[F + S2B::T * e]);
                if (q < kF64PrimeBound)
                    inv_rows_tile<ArithF64, S1, S2>(raw, b, t, r, prow, q, lds, ctl.scratch + (size_t)job * G::N);
                else
                    inv_rows_tile<ArithInt, S1, S2>(raw, b, t, r, prow, q, reinterpret_cast<uint64_t *>(lds), ctl.scratch + (size_t)job * G::N);
            }
            fused_publish(ctl.done + job);
        } else if (!skip) {
            fused_wait(ctl.done + job, n1, ctl.flags);
            const uint32_t c = threadIdx.x % kCols, F = threadIdx.x / kCols;
            const uint64_t *scol = ctl.scratch + (size_t)job * G::N + r.tile * kCols;
            uint64_t raw[S1B::E];
#pragma unroll
            for (int e = 0; e < S1B::E; e++) raw[e] = scol[(size_t)(F * S1B::E + e) * G::N2 + c];
            if (q < kF64PrimeBound)
                inv_cols_tile<ArithF64, S1, S2>(raw, b, t, r, prow, q, lds, b.dst + r.m * b.dstride + (size_t)r.l * G::N);
            else
                inv_cols_tile<ArithInt, S1, S2>(raw, b, t, r, prow, q, reinterpret_cast<uint64_t *>(lds), b.dst + r.m * b.dstride + (size_t)r.l * G::N);
        }
        __syncthreads();
    }
}

static __global__ void k_zero_u32(uint32_t *p, uint32_t n) {
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0;
}

}  // namespace pfa
