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

// Forward rounds with the twiddle values read from a per-row table instead of
// derived: tab[(2^g - 1) + j] holds the value rows_tw derives for stage g,
// index j < 2^g (2^S - 1 entries per row; see build_row_tab); the pair is
// completed by pair_of, so the butterflies see the derived twiddles exactly.
template <int S>
__device__ __forceinline__ void fwd_round_a_tab(double (&x)[Sub<S>::E], const ArithF64 &ar, const double *tab) {
    constexpr int LE = Sub<S>::LE, E = Sub<S>::E;
#pragma unroll
    for (int g = 0; g < LE; g++) {
        const int d = E >> (g + 1);
        ulonglong2 w[1 << (LE - 1)];
#pragma unroll
        for (int i = 0; i < (1 << g); i++) w[i] = ar.pair_of(tab[(1 << g) - 1 + i]);
#pragma unroll
        for (int e = 0; e < E; e++) {
            if (e & d) continue;
            ar.ct(x[e], x[e + d], w[e >> (LE - g)]);
        }
    }
}

template <int S>
__device__ __forceinline__ void fwd_round_b_tab(double (&x)[Sub<S>::E], const ArithF64 &ar, const double *tab,
                                                uint32_t F) {
    constexpr int LE = Sub<S>::LE, E = Sub<S>::E;
#pragma unroll
    for (int g = LE; g < S; g++) {
        const int d = 1 << (S - 1 - g);
        const uint32_t jb = F << (LE - S + g);
        ulonglong2 w[1 << (LE - 1)];
#pragma unroll
        for (int i = 0; i < (1 << (g + LE - S)); i++) w[i] = ar.pair_of(tab[(1 << g) - 1 + jb + i]);
#pragma unroll
        for (int e = 0; e < E; e++) {
            if (e & d) continue;
            ar.ct(x[e], x[e + d], w[e >> (S - g)]);
        }
    }
}

// Fills tab[row][(2^g - 1) + j] (rows of 2^S - 1 doubles) for rows 0 .. R-1 of
// a tile with the twiddle values rows_tw derives from the staged base factors
// rb[g * R + row] and small table, threads `tid` of `nthreads` sharing the work.
template <int S, int R>
__device__ __forceinline__ void build_row_tab(double *tab, const ArithF64 &ar, const ulonglong2 *rb,
                                              const ulonglong2 *small, uint32_t tid, uint32_t nthreads) {
    constexpr uint32_t PER = (1u << S) - 1;
    for (uint32_t e = tid; e < R * PER; e += nthreads) {
        const uint32_t row = e / PER, idx = e % PER;
        const uint32_t g = 31 - __builtin_clz(idx + 1), j = idx + 1 - (1u << g);
        const ulonglong2 B = rb[g * R + row];
        tab[e] = j == 0 ? ArithF64::as_f(B.x) : ar.twval(B, small[j]);
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
// walks tiles blockIdx.x, blockIdx.x + gridDim.x, ...; the inverse passes
// prefetch the next tile's residues into registers while they transform the
// current one, the forward passes run more workgroups instead.
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

// ================================================================ twiddles
// Where a tile's twiddle factors come from.  Columns passes index col[0 .. N1-1]
// (entries 1 .. N1-1 of the prime's table).  Rows passes index, in the integer
// policy, the prime's full table `full` at base N1 + k1, and in the FP64 policy
// the base factors rb[g * RBS + rrow] and the small table `small`.  The
// persistent two-pass kernels stage the entries a tile needs in LDS (RBS =
// ROWS, rrow = the row within the tile); other callers read the global tables
// (RBS = N1, rrow = k1).
struct TileTw {
    const ulonglong2 *col;
    const ulonglong2 *full;
    const ulonglong2 *rb;
    const ulonglong2 *small;
    uint32_t rrow;
};

template <int S1, int S2>
__device__ __forceinline__ TileTw global_tw(const NttTables &t, uint32_t prow, uint32_t k1, bool fwd) {
    using G = Geo<S1, S2>;
    const ulonglong2 *tab = (fwd ? t.tw : t.itw) + (size_t)prow * G::N;
    return TileTw{tab, tab, (fwd ? t.rb_fw : t.rb_inv) + (size_t)prow * S2 * G::N1,
                  (fwd ? t.small_fw : t.small_inv) + (size_t)prow * kSmall, k1};
}

// A gather of N twiddle entries into LDS, split in two so the caller can issue
// its data prefetch in between: global loads complete in issue order, so a load
// issued after the prefetch could not be waited for without waiting for the
// prefetch.  load() issues every thread's loads, store() writes them to LDS
// (the caller then synchronizes the workgroup).
template <int N, int THREADS>
struct TwStage {
    static constexpr int PER = (N + THREADS - 1) / THREADS;
    ulonglong2 v[PER];
    // every lane loads (surplus lanes a duplicate of the last entry): a load
    // under a branch would make the wait for it a wait for all loads
    template <class Src>
    __device__ __forceinline__ void load(Src src) {
#pragma unroll
        for (int p = 0; p < PER; p++) {
            const uint32_t i = threadIdx.x + p * THREADS;
            v[p] = src(i < (uint32_t)N ? i : (uint32_t)N - 1);
        }
    }
    __device__ __forceinline__ void store(ulonglong2 *dst) const {
#pragma unroll
        for (int p = 0; p < PER; p++) {
            const uint32_t i = threadIdx.x + p * THREADS;
            if (i < (uint32_t)N) dst[i] = v[p];
        }
    }
};

// Staged entries of a rows-pass tile: rb[g][tile ROWS + i] for g < S2, i < ROWS,
// then the small table's first 2^(S2-1) entries.
template <int S1, int S2, int R = Geo<S1, S2>::ROWS>
struct RowStage {
    using G = Geo<S1, S2>;
    static constexpr int RB = S2 * R;
    static constexpr int N = RB + (1 << (S2 - 1));
    TwStage<N, R * Sub<S2>::T> st;
    __device__ __forceinline__ void load(const NttTables &t, uint32_t prow, uint32_t tile, bool fwd) {
        const ulonglong2 *rb = (fwd ? t.rb_fw : t.rb_inv) + (size_t)prow * S2 * G::N1 + tile * R;
        const ulonglong2 *small = (fwd ? t.small_fw : t.small_inv) + (size_t)prow * kSmall;
        st.load([&](uint32_t i) { return i < (uint32_t)RB ? rb[(i / R) * G::N1 + i % R] : small[i - RB]; });
    }
    // LDS copy -> the tile's twiddle view (full: the prime's global table, for
    // the integer policy)
    __device__ __forceinline__ static TileTw view(const ulonglong2 *lds, const ulonglong2 *full, uint32_t rr) {
        return TileTw{nullptr, full, lds, lds + RB, rr};
    }
};

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
// (F E + e) of the column in the intermediate form (lazy).  tw: the prime's
// table (entries 1 .. N1-1 are read).
template <class A, int S1, int S2>
__device__ __forceinline__ void fwd_cols_core(typename A::T (&x)[Sub<S1>::E], const A &ar, const ulonglong2 *tw,
                                              typename A::T *lds) {
    using SB = Sub<S1>;
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

// store of fwd_cols_core's output into limb olimb (intermediate form); NT
// selects streaming stores (plain stores keep the lines in L2 for a consumer
// in the same launch)
template <class A, int S1, int S2, bool NT = true>
__device__ __forceinline__ void fwd_cols_store(const typename A::T (&x)[Sub<S1>::E], const A &ar, uint32_t tile,
                                               uint64_t *olimb) {
    using G = Geo<S1, S2>;
    using SB = Sub<S1>;
    uint64_t *dst = olimb + tile * kCols;
    const uint32_t c = threadIdx.x % kCols, F = threadIdx.x / kCols;
#pragma unroll
    for (int e = 0; e < SB::E; e++) {
        uint64_t *p = &dst[(size_t)(F * SB::E + e) * G::N2 + c];
        if (NT)
            st_stream(p, ar.store_mid(x[e]));
        else
            *p = ar.store_mid(x[e]);
    }
}

template <class A, int S1, int S2, bool NT = true>
__device__ __forceinline__ void fwd_cols_tile(const uint64_t (&raw)[Sub<S1>::E], const ulonglong2 *tw,
                                              const TileRef &r, uint64_t q, typename A::T *lds, uint64_t *olimb) {
    using SB = Sub<S1>;
    using T = typename A::T;
    const A ar(q);
    T x[SB::E];
#pragma unroll
    for (int e = 0; e < SB::E; e++) x[e] = ar.load(raw[e]);
    fwd_cols_core<A, S1, S2>(x, ar, tw, lds);
    fwd_cols_store<A, S1, S2, NT>(x, ar, r.tile, olimb);
}

// The forward passes keep no register prefetch: without it they fit 4 waves
// per SIMD (102 / 126 VGPRs, against 135 / 158 with a prefetched tile at 3),
// and the extra resident workgroups hide the load latency better (measured on
// the 2 x 35-limb config-2 batch: 43-44.5 -> 40.8-41 us per forward NTT).
template <int S1, int S2>
__global__ void __launch_bounds__((Geo<S1, S2>::COL_THREADS)) __attribute__((amdgpu_waves_per_eu(4, 8)))
ntt_fwd_cols(NttBatch b, NttTables t) {
    using G = Geo<S1, S2>;
    using SB = Sub<S1>;
    __shared__ double lds[G::COL_LDS];
    // the tile's twiddle factors (entries 1 .. N1-1 of its prime's table),
    // requested before its residues and staged in LDS: one wait covers both,
    // and the rounds read LDS instead of L1/L2 (config-2 forward NTT
    // 39.4-39.9 -> 37.4-38.0 us)
    __shared__ ulonglong2 twl[G::N1];
    const uint32_t total = b.M * b.L * G::COL_TILES;
    const uint32_t c = threadIdx.x % kCols, F = threadIdx.x / kCols;
    for (uint32_t cur = next_tile(b, G::COL_TILES, blockIdx.x, total); cur < total;
         cur = next_tile(b, G::COL_TILES, cur + gridDim.x, total)) {
        const TileRef r = decode_tile(b, G::COL_TILES, cur);
        const uint32_t prow = b.map.row(r.l);
        TwStage<G::N1, G::COL_THREADS> st;
        st.load([&](uint32_t i) { return t.tw[(size_t)prow * G::N + i]; });
        uint64_t raw[SB::E];
        const uint64_t *s = cols_src<S1, S2>(b, r, b.src, b.sstride);
#pragma unroll
        for (int e = 0; e < SB::E; e++) raw[e] = ld_stream(&s[(size_t)(F + SB::T * e) * G::N2 + c]);
        st.store(twl);
        __syncthreads();
        const uint64_t q = t.mod[prow];
        const ulonglong2 *tw = twl;
        uint64_t *olimb = b.dst + r.m * b.dstride + (size_t)r.l * G::N;
        if (q < kF64PrimeBound)
            fwd_cols_tile<ArithF64, S1, S2>(raw, tw, r, q, lds, olimb);
        else
            fwd_cols_tile<ArithInt, S1, S2>(raw, tw, r, q, reinterpret_cast<uint64_t *>(lds), olimb);
        __syncthreads();
    }
}

// Rows pass: dst (intermediate) -> dst (canonical).
// Forward rows pass of one tile row k1.  In: x[e] = element (F + T e) of the
// row in the intermediate form.  Out: x[e] = element (F + T e) of the
// transformed row (lazy; the final LDS transpose makes stores coalesced).
// The caller separates consecutive calls on the same LDS with a barrier.
template <class A, int S1, int S2, int RBS>
__device__ __forceinline__ void fwd_rows_core(typename A::T (&x)[Sub<S2>::E], const A &ar, const TileTw &w,
                                              uint32_t k1, typename A::T *lr) {
    using G = Geo<S1, S2>;
    using SB = Sub<S2>;
    const uint32_t F = threadIdx.x % SB::T;
    if constexpr (A::kF64)
        fwd_round_a_derived<S2, RBS>(x, ar, w.rb, w.small, w.rrow);
    else
        fwd_round_a<A, S2>(x, ar, w.full, G::N1 + k1);
#pragma unroll
    for (int e = 0; e < SB::E; e++) {
        ar.reduce(x[e]);
        lr[rpad(F + SB::T * e)] = x[e];
    }
    __syncthreads();
#pragma unroll
    for (int e = 0; e < SB::E; e++) x[e] = lr[rpad(F * SB::E + e)];
    if constexpr (A::kF64)
        fwd_round_b_derived<S2, RBS>(x, ar, w.rb, w.small, w.rrow, F);
    else
        fwd_round_b<A, S2>(x, ar, w.full, G::N1 + k1, F);
    __syncthreads();
#pragma unroll
    for (int e = 0; e < SB::E; e++) lr[rpad(F * SB::E + e)] = x[e];
    __syncthreads();
#pragma unroll
    for (int e = 0; e < SB::E; e++) x[e] = lr[rpad(F + SB::T * e)];
}

// the same with the twiddles read from the global tables
template <class A, int S1, int S2>
__device__ __forceinline__ void fwd_rows_core(typename A::T (&x)[Sub<S2>::E], const A &ar, const NttTables &t,
                                              uint32_t prow, uint32_t k1, typename A::T *lr) {
    fwd_rows_core<A, S1, S2, Geo<S1, S2>::N1>(x, ar, global_tw<S1, S2>(t, prow, k1, true), k1, lr);
}

template <class A, int S1, int S2, int RBS, int R = Geo<S1, S2>::ROWS>
__device__ __forceinline__ void fwd_rows_tile(const uint64_t (&raw)[Sub<S2>::E], const TileTw &w, const TileRef &r,
                                              uint64_t q, typename A::T *lds, uint64_t *olimb) {
    using G = Geo<S1, S2>;
    using SB = Sub<S2>;
    using T = typename A::T;
    const A ar(q);
    const uint32_t F = threadIdx.x % SB::T, rr = threadIdx.x / SB::T;
    const uint32_t k1 = r.tile * R + rr;
    uint64_t *rowp = olimb + (size_t)k1 * G::N2;
    T x[SB::E];
#pragma unroll
    for (int e = 0; e < SB::E; e++) x[e] = ar.load_mid(raw[e]);
    fwd_rows_core<A, S1, S2, RBS>(x, ar, w, k1, lds + rr * G::ROW_PITCH);
#pragma unroll
    for (int e = 0; e < SB::E; e++) st_stream(&rowp[F + SB::T * e], ar.store(x[e]));
}

template <int S1, int S2, int R = Geo<S1, S2>::ROWS>
__device__ __forceinline__ const uint64_t *rows_ptr(const NttBatch &b, const TileRef &r, const uint64_t *base,
                                                    uint64_t stride) {
    using G = Geo<S1, S2>;
    const uint32_t rr = threadIdx.x / Sub<S2>::T;
    return base + r.m * stride + (size_t)r.l * G::N + (size_t)(r.tile * R + rr) * G::N2;
}

template <int S1, int S2, int R = Geo<S1, S2>::ROWS>
__global__ void __launch_bounds__(R * Sub<S2>::T) __attribute__((amdgpu_waves_per_eu(4, 8)))
ntt_fwd_rows(NttBatch b, NttTables t) {
    using G = Geo<S1, S2>;
    using SB = Sub<S2>;
    using RS = RowStage<S1, S2, R>;
    constexpr uint32_t TILES = G::N1 / R;
    __shared__ double lds[R * G::ROW_PITCH];
    __shared__ ulonglong2 twl[RS::N];
    const uint32_t total = b.M * b.L * TILES;
    const uint32_t F = threadIdx.x % SB::T, rr = threadIdx.x / SB::T;
    for (uint32_t cur = next_tile(b, TILES, blockIdx.x, total); cur < total;
         cur = next_tile(b, TILES, cur + gridDim.x, total)) {
        const TileRef r = decode_tile(b, TILES, cur);
        const uint32_t prow = b.map.row(r.l);
        const uint64_t q = t.mod[prow];
        // the tile's twiddles are requested before its residues, so both are
        // in flight together and staged in LDS once
        RS stage;
        stage.load(t, prow, r.tile, true);
        uint64_t raw[SB::E];
        const uint64_t *s = rows_ptr<S1, S2, R>(b, r, b.src, b.sstride);
#pragma unroll
        for (int e = 0; e < SB::E; e++) raw[e] = ld_stream(&s[F + SB::T * e]);
        stage.st.store(twl);
        __syncthreads();
        const TileTw w = RS::view(twl, t.tw + (size_t)prow * G::N, rr);
        uint64_t *olimb = b.dst + r.m * b.dstride + (size_t)r.l * G::N;
        if (q < kF64PrimeBound)
            fwd_rows_tile<ArithF64, S1, S2, R, R>(raw, w, r, q, lds, olimb);
        else
            fwd_rows_tile<ArithInt, S1, S2, R, R>(raw, w, r, q, reinterpret_cast<uint64_t *>(lds), olimb);
        __syncthreads();
    }
}

// ================================================================ inverse
// Rows pass first: src (canonical) -> dst (intermediate).
// The pass over a tile whose residues are in LDS already (element k of tile row
// rr at lds[rr ROW_PITCH + rpad(k)], as A::load gives it), after a barrier.
// With active false (whole waves beyond the tile's R T threads of a larger
// workgroup) a thread only takes part in the barriers.
template <class A, int S1, int S2, int RBS, bool NT = true, int R = Geo<S1, S2>::ROWS>
__device__ __forceinline__ void inv_rows_lds(const TileTw &w, const TileRef &r, uint64_t q, typename A::T *lds,
                                             uint64_t *olimb, bool active = true) {
    using G = Geo<S1, S2>;
    using SB = Sub<S2>;
    using T = typename A::T;
    const A ar(q);
    const uint32_t F = threadIdx.x % SB::T, rr = threadIdx.x / SB::T;
    const uint32_t k1 = r.tile * R + rr;
    uint64_t *drow = olimb + (size_t)k1 * G::N2;
    T *lr = lds + rr * G::ROW_PITCH;
    T x[SB::E];
    if (active) {
#pragma unroll
        for (int e = 0; e < SB::E; e++) x[e] = lr[rpad(F * SB::E + e)];
        if constexpr (A::kF64)
            inv_round_a_derived<S2, RBS>(x, ar, w.rb, w.small, w.rrow, F);
        else
            inv_round_a<A, S2>(x, ar, w.full, G::N1 + k1, F);
    }
    __syncthreads();
    if (active) {
#pragma unroll
        for (int e = 0; e < SB::E; e++) lr[rpad(F * SB::E + e)] = x[e];
    }
    __syncthreads();
    if (!active) return;
#pragma unroll
    for (int e = 0; e < SB::E; e++) x[e] = lr[rpad(F + SB::T * e)];
    if constexpr (A::kF64)
        inv_round_b_derived<S2, RBS>(x, ar, w.rb, w.small, w.rrow);
    else
        inv_round_b<A, S2, false>(x, ar, w.full, G::N1 + k1, ulonglong2{0, 0});
#pragma unroll
    for (int e = 0; e < SB::E; e++) {
        if (NT)
            st_stream(&drow[F + SB::T * e], ar.store_mid(x[e]));
        else
            drow[F + SB::T * e] = ar.store_mid(x[e]);
    }
}

template <class A, int S1, int S2, int RBS, bool NT = true, int R = Geo<S1, S2>::ROWS>
__device__ __forceinline__ void inv_rows_tile(const uint64_t (&raw)[Sub<S2>::E], const TileTw &w, const TileRef &r,
                                              uint64_t q, typename A::T *lds, uint64_t *olimb) {
    using G = Geo<S1, S2>;
    using SB = Sub<S2>;
    const A ar(q);
    const uint32_t F = threadIdx.x % SB::T, rr = threadIdx.x / SB::T;
    typename A::T *lr = lds + rr * G::ROW_PITCH;
#pragma unroll
    for (int e = 0; e < SB::E; e++) lr[rpad(F + SB::T * e)] = ar.load(raw[e]);
    __syncthreads();
    inv_rows_lds<A, S1, S2, RBS, NT, R>(w, r, q, lds, olimb);
}

template <int S1, int S2, int R = Geo<S1, S2>::ROWS>
__global__ void __launch_bounds__(R * Sub<S2>::T) ntt_inv_rows(NttBatch b, NttTables t) {
    using G = Geo<S1, S2>;
    using SB = Sub<S2>;
    constexpr uint32_t TILES = G::N1 / R;
    __shared__ double lds[R * G::ROW_PITCH];
    const uint32_t total = b.M * b.L * TILES;
    const uint32_t F = threadIdx.x % SB::T, rr = threadIdx.x / SB::T;
    uint32_t cur = next_tile(b, TILES, blockIdx.x, total);
    uint64_t raw[SB::E];
    if (cur < total) {
        const uint64_t *s = rows_ptr<S1, S2, R>(b, decode_tile(b, TILES, cur), b.src, b.sstride);
#pragma unroll
        for (int e = 0; e < SB::E; e++) raw[e] = ld_stream(&s[F + SB::T * e]);
    }
    while (cur < total) {
        const uint32_t nxt = next_tile(b, TILES, cur + gridDim.x, total);
        const TileRef r = decode_tile(b, TILES, cur);
        uint64_t nraw[SB::E];
        if (nxt < total) {
            const uint64_t *s = rows_ptr<S1, S2, R>(b, decode_tile(b, TILES, nxt), b.src, b.sstride);
#pragma unroll
            for (int e = 0; e < SB::E; e++) nraw[e] = ld_stream(&s[F + SB::T * e]);
        }
        const uint32_t prow = b.map.row(r.l);
        const uint64_t q = t.mod[prow];
        const TileTw w = global_tw<S1, S2>(t, prow, r.tile * R + rr, false);
        uint64_t *olimb = b.dst + r.m * b.dstride + (size_t)r.l * G::N;
        if (q < kF64PrimeBound)
            inv_rows_tile<ArithF64, S1, S2, G::N1, true, R>(raw, w, r, q, lds, olimb);
        else
            inv_rows_tile<ArithInt, S1, S2, G::N1, true, R>(raw, w, r, q, reinterpret_cast<uint64_t *>(lds), olimb);
#pragma unroll
        for (int e = 0; e < SB::E; e++) raw[e] = nraw[e];
        cur = nxt;
        __syncthreads();
    }
}

// The same pass without register prefetch, its tile's twiddle factors staged
// in LDS (requested before the residues, so one wait covers both) instead of
// read from the global tables inside the rounds: 142 VGPRs, 3 waves per SIMD.
// Faster on large batches (config-2 inverse 44.5-44.9 -> 41.3 us), slightly
// slower on the few-limb transforms of a key switch, so ntt_inverse picks it
// by batch size.
template <int S1, int S2, int R = Geo<S1, S2>::ROWS>
__global__ void __launch_bounds__(R * Sub<S2>::T) __attribute__((amdgpu_waves_per_eu(3, 8)))
ntt_inv_rows_staged(NttBatch b, NttTables t) {
    using G = Geo<S1, S2>;
    using SB = Sub<S2>;
    using RS = RowStage<S1, S2, R>;
    constexpr uint32_t TILES = G::N1 / R;
    __shared__ double lds[R * G::ROW_PITCH];
    __shared__ ulonglong2 twl[RS::N];
    const uint32_t total = b.M * b.L * TILES;
    const uint32_t F = threadIdx.x % SB::T, rr = threadIdx.x / SB::T;
    for (uint32_t cur = next_tile(b, TILES, blockIdx.x, total); cur < total;
         cur = next_tile(b, TILES, cur + gridDim.x, total)) {
        const TileRef r = decode_tile(b, TILES, cur);
        const uint32_t prow = b.map.row(r.l);
        const uint64_t q = t.mod[prow];
        RS stage;
        stage.load(t, prow, r.tile, false);
        uint64_t raw[SB::E];
        const uint64_t *s = rows_ptr<S1, S2, R>(b, r, b.src, b.sstride);
#pragma unroll
        for (int e = 0; e < SB::E; e++) raw[e] = ld_stream(&s[F + SB::T * e]);
        stage.st.store(twl);
        __syncthreads();
        const TileTw w = RS::view(twl, t.itw + (size_t)prow * G::N, rr);
        uint64_t *olimb = b.dst + r.m * b.dstride + (size_t)r.l * G::N;
        if (q < kF64PrimeBound)
            inv_rows_tile<ArithF64, S1, S2, R, true, R>(raw, w, r, q, lds, olimb);
        else
            inv_rows_tile<ArithInt, S1, S2, R, true, R>(raw, w, r, q, reinterpret_cast<uint64_t *>(lds), olimb);
        __syncthreads();
    }
}

// Columns pass: dst (intermediate) -> dst (canonical), N^-1 and, when scale is
// not null, the limb's scale pair, read only after the rounds: held in
// registers from the tile's start it made the pass spill (127 VGPRs and 12
// bytes of scratch per lane at 4 waves per SIMD; config-2 inverse +2.2 us), and
// read with scalar loads at the start the pass was slower still (+4.5 us).
template <class A, int S1, int S2>
__device__ __forceinline__ void inv_cols_tile(const uint64_t (&raw)[Sub<S1>::E], const ulonglong2 *itw,
                                              ulonglong2 ninv, const ulonglong2 *scale, const TileRef &r,
                                              uint64_t q, typename A::T *lds, uint64_t *olimb) {
    using G = Geo<S1, S2>;
    using SB = Sub<S1>;
    using T = typename A::T;
    const A ar(q);
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
    inv_round_b<A, S1, true>(x, ar, itw, 1, ninv);
    if (scale) {
        const ulonglong2 sc = *scale;
#pragma unroll
        for (int e = 0; e < SB::E; e++) ar.mul(x[e], sc);
    }
#pragma unroll
    for (int e = 0; e < SB::E; e++) st_stream(&data[(size_t)(F + SB::T * e) * G::N2 + c], ar.store(x[e]));
}

// Like the forward columns pass: no register prefetch (124 VGPRs, 4 waves
// per SIMD) and the tile's twiddle factors staged in LDS, requested before its
// residues (config-2 inverse 41.0-41.2 -> 39.4 us; with the prefetch at 3
// waves, the staging alone had cost 3 us).
template <int S1, int S2>
__global__ void __launch_bounds__((Geo<S1, S2>::COL_THREADS)) __attribute__((amdgpu_waves_per_eu(4, 8)))
ntt_inv_cols(NttBatch b, NttTables t) {
    using G = Geo<S1, S2>;
    using SB = Sub<S1>;
    __shared__ double lds[G::COL_LDS];
    __shared__ ulonglong2 twl[G::N1];
    const uint32_t total = b.M * b.L * G::COL_TILES;
    const uint32_t c = threadIdx.x % kCols, F = threadIdx.x / kCols;
    for (uint32_t cur = next_tile(b, G::COL_TILES, blockIdx.x, total); cur < total;
         cur = next_tile(b, G::COL_TILES, cur + gridDim.x, total)) {
        const TileRef r = decode_tile(b, G::COL_TILES, cur);
        const uint32_t prow = b.map.row(r.l);
        TwStage<G::N1, G::COL_THREADS> st;
        st.load([&](uint32_t i) { return t.itw[(size_t)prow * G::N + i]; });
        uint64_t raw[SB::E];
        const uint64_t *s = cols_src<S1, S2>(b, r, b.src, b.sstride);
#pragma unroll
        for (int e = 0; e < SB::E; e++) raw[e] = ld_stream(&s[(size_t)(F * SB::E + e) * G::N2 + c]);
        st.store(twl);
        __syncthreads();
        const uint64_t q = t.mod[prow];
        const ulonglong2 *sc = b.scale ? b.scale + r.l : nullptr;
        uint64_t *olimb = b.dst + r.m * b.dstride + (size_t)r.l * G::N;
        if (q < kF64PrimeBound)
            inv_cols_tile<ArithF64, S1, S2>(raw, twl, t.ninv[prow], sc, r, q, lds, olimb);
        else
            inv_cols_tile<ArithInt, S1, S2>(raw, twl, t.ninv[prow], sc, r, q, reinterpret_cast<uint64_t *>(lds),
                                            olimb);
        __syncthreads();
    }
}

}  // namespace pfa

namespace pfa {

// ================================================================ single launch
// One launch runs both passes of every limb of the batch, and a limb's
// intermediate never leaves the L2 of the XCD that transforms it: HBM sees one
// read of the input and one write of the output instead of two of each.
//
// Jobs (j = l M + m) belong to XCD j mod 8.  Every workgroup reads the id of
// the XCD it runs on (hardware register) and serves only that XCD's jobs, so a
// job's two passes always share one L2 whatever the dispatch order.  (The
// device deals a launch's workgroups to the 8 XCDs round-robin, starting at an
// XCD that depends on earlier dispatches, so a grid that is a multiple of 8
// gives every XCD the same number of workgroups.)  Work is handed out
// dynamically per XCD:
//   - first-pass tiles by a ticket counter in job order, at most `window` jobs
//     ahead of the oldest job whose second pass is not fully handed out (the
//     front), which bounds the limbs held in L2;
//   - second-pass tiles of a job once all its first-pass tiles are finished,
//     by a per-job claim counter.
// A workgroup waits only when no tile can be handed to it; then every
// first-pass tile of the jobs in the window is held by a running workgroup,
// which finishes it without waiting, so every wait ends (no co-residency or
// cooperative launch is assumed).  A wait is still bounded in time: on expiry
// the workgroup records the error (device word and a mapped host word) and
// leaves, and the kernel ends.  The last workgroup to leave checks that every
// tile of the batch was transformed (a device-wide count) and records an error
// otherwise, so missing work can never pass silently.
//
// Visibility inside an XCD: a first-pass tile's stores are complete in L2
// (s_waitcnt vmcnt(0)) before its job's finished count is raised; a workgroup
// that starts a second-pass tile invalidates its CU's L1 (buffer_inv sc0) and
// reads the limb from the XCD's L2.
//
// Control words live in two blocks per (context, thread, stream): a launch
// uses one (all zero at launch) and zeroes the part of the other that the
// previous launch used, for the next launch.
constexpr uint32_t kXcds = 8;
constexpr uint32_t kFlowXcdWords = 64;   // per XCD: first-pass ticket at +0, front at +32 (own 128-B lines)
// after the XCD words, one 128-B line whose first 8 bytes count, for the whole
// launch, (workgroups that left) << 32 | (tiles transformed)
constexpr uint32_t kFlowHeadWords = kXcds * kFlowXcdWords + 32;
constexpr uint32_t kFlowJobWords = 16;   // per job: finished first-pass tiles at +0, second-pass claims at +1
constexpr uint32_t kFlowMaxJobs = 4096;
constexpr uint32_t kFlowBlockWords = kFlowHeadWords + kFlowMaxJobs * kFlowJobWords;
constexpr uint32_t kFlowMaxWindow = 32;
// error bits
constexpr uint32_t kFlowErrWait = 1u;        // a wait expired
constexpr uint32_t kFlowErrIncomplete = 2u;  // the launch ended with tiles not transformed

struct FlowCtl {
    uint32_t *blk;         // this launch's control block (zero at launch)
    uint32_t *other;       // the other block: its first other_jobs jobs are zeroed here
    uint32_t other_jobs;
    uint32_t window;       // 1 .. kFlowMaxWindow
    uint32_t wait_ticks;   // bound of one wait, s_memrealtime ticks (100 MHz)
    uint32_t *host_err;    // mapped pinned host word: the error bits are stored there, on error only
};

template <int S1, int S2>
struct FlowGeo {
    using G = Geo<S1, S2>;
    static constexpr bool OK = G::COL_THREADS == 256 && G::ROW_THREADS == 256 && G::COL_TILES == G::ROW_TILES;
    static constexpr uint32_t T = G::COL_TILES;
    static constexpr int LDS = G::COL_LDS > G::ROW_LDS ? G::COL_LDS : G::ROW_LDS;
    static constexpr int TWL = G::N1 > RowStage<S1, S2>::N ? G::N1 : RowStage<S1, S2>::N;
};

// The XCD-local hand-offs of this library (the single-launch NTT's second
// pass below, the key-switch inner product's split items in fused_ks.hip) rely
// on the cache behaviour of gfx942 / gfx950: a CU's L1 is write-through, each
// XCD has one L2 that all its CUs share, and a vector store stays counted by
// vmcnt until that L2 holds it.  So data a workgroup stored and waited for
// (s_waitcnt vmcnt(0)) before a relaxed agent-scope atomic is in its XCD's L2
// when another workgroup of the same XCD sees that atomic, and the reader gets
// it after dropping its own CU's L1 (buffer_inv sc0).  That is not ordering the
// HIP memory model guarantees; other targets would need release / acquire
// fences, so they are refused here.
#if defined(__HIP_DEVICE_COMPILE__) && !defined(__gfx942__) && !defined(__gfx950__)
#error "the XCD-local hand-offs assume the gfx942 / gfx950 cache hierarchy"
#endif

__device__ __forceinline__ uint32_t xcc_id() {
    uint32_t v;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
    return v & 0xfu;
}

// Reads of control words are read-modify-writes: they execute in the XCD's L2
// where the words live, and never hit a stale L1 line.
__device__ __forceinline__ uint32_t flow_rd(uint32_t *p) {
    return __hip_atomic_fetch_or(p, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t flow_add(uint32_t *p, uint32_t v) {
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void flow_error(const FlowCtl &c, uint32_t bits) {
    __hip_atomic_store(c.host_err, bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

constexpr uint32_t kFlowExit = 0xffffffffu, kFlowWait = 0xfffffffeu, kFlowPass2 = 0x80000000u;

// Next command of a workgroup, decided by wave 0 (every lane of it calls this):
// a first-pass tile k (local job k / T, tile k mod T), kFlowPass2 | k for a
// second-pass tile, kFlowWait or kFlowExit.  Lane i looks at job front + i.
template <uint32_t T>
__device__ __forceinline__ uint32_t flow_decide(const FlowCtl &c, uint32_t x, uint32_t nj, uint32_t *next1,
                                                uint32_t *front, uint32_t *jobw) {
    const uint32_t lane = threadIdx.x;
    uint32_t f = lane == 0 ? flow_rd(front) : 0u;
    f = __builtin_amdgcn_readfirstlane(f);
    if (f >= nj) return kFlowExit;
    const uint32_t lj = f + lane;
    const bool act = lane < c.window && lj < nj;
    uint32_t *jw = jobw + (size_t)(x + kXcds * lj) * kFlowJobWords;
    uint32_t done = 0, claimed = T;
    if (act) {
        done = flow_rd(jw);
        claimed = flow_rd(jw + 1);
    }
    // advance the front past leading jobs whose second pass is fully handed out
    // (a failed exchange means another workgroup moved it; either is fine)
    const uint64_t full = __ballot(act && claimed >= T);
    const uint32_t adv = (uint32_t)__builtin_ctzll(~full);
    if (adv > 0 && lane == 0) {
        uint32_t expect = f;
        __hip_atomic_compare_exchange_strong(front, &expect, f + adv, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
    }
    if (f + adv >= nj) return kFlowExit;
    uint64_t ready = __ballot(act && done >= T && claimed < T);
    while (ready) {
        const uint32_t i = (uint32_t)__builtin_ctzll(ready);
        ready &= ready - 1;
        uint32_t k = 0;
        if (lane == 0) k = flow_add(jobw + (size_t)(x + kXcds * (f + i)) * kFlowJobWords + 1, 1u);
        k = __builtin_amdgcn_readfirstlane(k);
        if (k < T) return kFlowPass2 | ((f + i) * T + k);
    }
    uint32_t k1 = kFlowWait;
    if (lane == 0) {
        const uint32_t n1 = nj * T;
        uint32_t k = flow_rd(next1);
        if (k < n1 && k / T < f + c.window) {
            k = flow_add(next1, 1u);
            if (k < n1) k1 = k;
        }
    }
    return __builtin_amdgcn_readfirstlane(k1);
}

// Tiles of one job for the single-launch kernel.  FWD: columns pass then rows
// pass; inverse: rows pass then columns pass.  twl: LDS for the tile's staged
// twiddle factors, lds: the transpose buffer.
template <bool FWD, int S1, int S2>
struct FlowJob {
    using G = Geo<S1, S2>;
    using S1B = Sub<S1>;
    using S2B = Sub<S2>;
    using RS = RowStage<S1, S2>;
    const NttBatch &b;
    const NttTables &t;
    uint32_t m, l, prow;
    uint64_t q;
    uint64_t *limb;

    __device__ FlowJob(const NttBatch &b_, const NttTables &t_, uint32_t job) : b(b_), t(t_) {
        m = job % b.M;
        l = job / b.M;
        prow = b.map.row(l);
        q = t.mod[prow];
        limb = b.dst + m * b.dstride + (size_t)l * G::N;
    }

    // first-pass tile: source -> the tile's part of the output limb in the
    // intermediate form, with plain stores so the lines stay in L2
    __device__ void first(uint32_t tile, double *lds, ulonglong2 *twl) const {
        const TileRef r{m, l, tile};
        if (FWD) {
            const uint32_t c = threadIdx.x % kCols, F = threadIdx.x / kCols;
            TwStage<G::N1, G::COL_THREADS> st;
            st.load([&](uint32_t i) { return t.tw[(size_t)prow * G::N + i]; });
            const uint64_t *s = cols_src<S1, S2>(b, r, b.src, b.sstride);
            uint64_t raw[S1B::E];
#pragma unroll
            for (int e = 0; e < S1B::E; e++) raw[e] = ld_stream(&s[(size_t)(F + S1B::T * e) * G::N2 + c]);
            st.store(twl);
            __syncthreads();
            if (q < kF64PrimeBound)
                fwd_cols_tile<ArithF64, S1, S2, false>(raw, twl, r, q, lds, limb);
            else
                fwd_cols_tile<ArithInt, S1, S2, false>(raw, twl, r, q, reinterpret_cast<uint64_t *>(lds), limb);
        } else {
            const uint32_t F = threadIdx.x % S2B::T, rr = threadIdx.x / S2B::T;
            RS stage;
            stage.load(t, prow, tile, false);
            const uint64_t *s = rows_ptr<S1, S2>(b, r, b.src, b.sstride);
            uint64_t raw[S2B::E];
#pragma unroll
            for (int e = 0; e < S2B::E; e++) raw[e] = ld_stream(&s[F + S2B::T * e]);
            stage.st.store(twl);
            __syncthreads();
            const TileTw w = RS::view(twl, t.itw + (size_t)prow * G::N, rr);
            if (q < kF64PrimeBound)
                inv_rows_tile<ArithF64, S1, S2, G::ROWS, false>(raw, w, r, q, lds, limb);
            else
                inv_rows_tile<ArithInt, S1, S2, G::ROWS, false>(raw, w, r, q, reinterpret_cast<uint64_t *>(lds),
                                                                limb);
        }
    }

    // second-pass tile of the output limb, after all first-pass tiles of the job
    __device__ void second(uint32_t tile, double *lds, ulonglong2 *twl) const {
        asm volatile("buffer_inv sc0" ::: "memory");
        const TileRef r{m, l, tile};
        if (FWD) {
            const uint32_t F = threadIdx.x % S2B::T, rr = threadIdx.x / S2B::T;
            RS stage;
            stage.load(t, prow, tile, true);
            const uint64_t *s = rows_ptr<S1, S2>(b, r, b.dst, b.dstride);
            uint64_t raw[S2B::E];
#pragma unroll
            for (int e = 0; e < S2B::E; e++) raw[e] = s[F + S2B::T * e];
            stage.st.store(twl);
            __syncthreads();
            const TileTw w = RS::view(twl, t.tw + (size_t)prow * G::N, rr);
            if (q < kF64PrimeBound)
                fwd_rows_tile<ArithF64, S1, S2, G::ROWS>(raw, w, r, q, lds, limb);
            else
                fwd_rows_tile<ArithInt, S1, S2, G::ROWS>(raw, w, r, q, reinterpret_cast<uint64_t *>(lds), limb);
        } else {
            const uint32_t c = threadIdx.x % kCols, F = threadIdx.x / kCols;
            TwStage<G::N1, G::COL_THREADS> st;
            st.load([&](uint32_t i) { return t.itw[(size_t)prow * G::N + i]; });
            const uint64_t *s = cols_src<S1, S2>(b, r, b.dst, b.dstride);
            uint64_t raw[S1B::E];
#pragma unroll
            for (int e = 0; e < S1B::E; e++) raw[e] = s[(size_t)(F * S1B::E + e) * G::N2 + c];
            st.store(twl);
            __syncthreads();
            const ulonglong2 *sc = b.scale ? b.scale + l : nullptr;
            if (q < kF64PrimeBound)
                inv_cols_tile<ArithF64, S1, S2>(raw, twl, t.ninv[prow], sc, r, q, lds, limb);
            else
                inv_cols_tile<ArithInt, S1, S2>(raw, twl, t.ninv[prow], sc, r, q, reinterpret_cast<uint64_t *>(lds),
                                                limb);
        }
    }
};

template <bool FWD, int S1, int S2>
__device__ __forceinline__ void flow_run(const NttBatch &b, const NttTables &t, const FlowCtl &c) {
    using FG = FlowGeo<S1, S2>;
    constexpr uint32_t T = FG::T;
    __shared__ double lds[FG::LDS];
    __shared__ ulonglong2 twl[FG::TWL];
    __shared__ uint32_t s_cmd;
    {
        const uint32_t words = kFlowHeadWords + c.other_jobs * kFlowJobWords;
        for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < words; i += gridDim.x * blockDim.x)
            c.other[i] = 0u;
    }
    const uint32_t x = xcc_id() & (kXcds - 1);
    const uint32_t J = b.M * b.L;
    const uint32_t nj = J > x ? (J - x + kXcds - 1) / kXcds : 0u;
    uint32_t *next1 = c.blk + x * kFlowXcdWords, *front = next1 + 32;
    uint32_t *jobw = c.blk + kFlowHeadWords;
    uint64_t wait_from = 0;
    bool waiting = false;
    uint32_t tiles = 0;  // tiles this workgroup transformed (or skipped as excluded)
    for (;;) {
        if (threadIdx.x < 64) {
            uint32_t cmd = flow_decide<T>(c, x, nj, next1, front, jobw);
            if (threadIdx.x == 0) {
                if (cmd == kFlowWait) {
                    const uint64_t now = __builtin_amdgcn_s_memrealtime();
                    if (!waiting) {
                        waiting = true;
                        wait_from = now;
                    } else if (now - wait_from > c.wait_ticks) {
                        flow_error(c, kFlowErrWait);
                        cmd = kFlowExit;
                    }
                } else {
                    waiting = false;
                }
                s_cmd = cmd;
            }
        }
        __syncthreads();
        const uint32_t cmd = s_cmd;
        __syncthreads();
        if (cmd == kFlowExit) break;
        if (cmd == kFlowWait) {
            __builtin_amdgcn_s_sleep(2);
            continue;
        }
        const uint32_t k = cmd & ~kFlowPass2;
        const uint32_t job = x + kXcds * (k / T);
        const FlowJob<FWD, S1, S2> fj(b, t, job);
        const bool skip = b.excluded(fj.m, fj.l);
        if (cmd & kFlowPass2) {
            if (!skip) fj.second(k % T, lds, twl);
        } else {
            if (!skip) fj.first(k % T, lds, twl);
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            if (threadIdx.x == 0) flow_add(jobw + (size_t)job * kFlowJobWords, 1u);
        }
        ++tiles;
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        uint64_t *fin = reinterpret_cast<uint64_t *>(c.blk + kXcds * kFlowXcdWords);
        const uint64_t old = __hip_atomic_fetch_add(fin, (1ull << 32) | tiles, __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT);
        if ((uint32_t)(old >> 32) == gridDim.x - 1 && (uint32_t)old + tiles != 2u * T * J)
            flow_error(c, kFlowErrIncomplete);
    }
}

template <int S1, int S2, int W>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(W, 8)))
ntt_fwd_flow(NttBatch b, NttTables t, FlowCtl c) {
    static_assert(FlowGeo<S1, S2>::OK, "single-launch NTT needs matching 256-thread passes");
    flow_run<true, S1, S2>(b, t, c);
}

template <int S1, int S2, int W>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(W, 8)))
ntt_inv_flow(NttBatch b, NttTables t, FlowCtl c) {
    static_assert(FlowGeo<S1, S2>::OK, "single-launch NTT needs matching 256-thread passes");
    flow_run<false, S1, S2>(b, t, c);
}

// Records XCD ids by workgroup (the probe that enables the single-launch path).
static __global__ void k_xcc_probe(uint32_t *out) {
    if (threadIdx.x == 0) out[blockIdx.x] = xcc_id();
}

}  // namespace pfa
