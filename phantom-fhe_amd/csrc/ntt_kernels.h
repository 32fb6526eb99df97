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
    const ulonglong2 *small_fw;  // [QP][16] psi^brv(i), i < 16
    const ulonglong2 *small_inv; // [QP][16] psi^-brv(i), i < 16 (no N^-1 fold)
};

// Twiddles whose index bits are disjoint factor: with brv additive on disjoint
// bits, tw[A + i] = psi^brv(A) psi^brv(i) = tw[A] * small[i] when the low bits
// of A that i occupies are zero.  The rows pass loads one table entry per stage
// and derives the others from a 16-entry table with one modular product each
// (FP64 policy), cutting its twiddle reads ~4x.

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

// Rows-pass rounds with derived twiddles (FP64 policy only).
// forward, stages g = 0 .. LE-1 on u = F + T e: index (base << g) + i, i = e >> (LE - g)
template <int S>
__device__ __forceinline__ void fwd_round_a_derived(double (&x)[Sub<S>::E], const ArithF64 &ar,
                                                    const ulonglong2 *tw, const ulonglong2 *small, uint32_t base) {
    constexpr int LE = Sub<S>::LE, E = Sub<S>::E;
#pragma unroll
    for (int g = 0; g < LE; g++) {
        const int d = E >> (g + 1);
        const ulonglong2 B = tw[base << g];
        ulonglong2 w[1 << (LE - 1)];
#pragma unroll
        for (int i = 0; i < (1 << g); i++) w[i] = i == 0 ? B : ar.twmul(B, small[i]);
#pragma unroll
        for (int e = 0; e < E; e++) {
            if (e & d) continue;
            ar.ct(x[e], x[e + d], w[e >> (LE - g)]);
        }
    }
}

// forward, stages g = LE .. S-1 on u = F' E + e: index (base << g) + (F' << (LE - S + g)) + i, i = e >> (S - g)
template <int S>
__device__ __forceinline__ void fwd_round_b_derived(double (&x)[Sub<S>::E], const ArithF64 &ar,
                                                    const ulonglong2 *tw, const ulonglong2 *small, uint32_t base,
                                                    uint32_t F) {
    constexpr int LE = Sub<S>::LE, E = Sub<S>::E;
#pragma unroll
    for (int g = LE; g < S; g++) {
        const int d = 1 << (S - 1 - g);
        const ulonglong2 B = tw[(base << g) + (F << (LE - S + g))];
        ulonglong2 w[1 << (LE - 1)];
#pragma unroll
        for (int i = 0; i < (1 << (g + LE - S)); i++) w[i] = i == 0 ? B : ar.twmul(B, small[i]);
#pragma unroll
        for (int e = 0; e < E; e++) {
            if (e & d) continue;
            ar.ct(x[e], x[e + d], w[e >> (S - g)]);
        }
    }
}

// inverse, stages g = S-1 .. LE on u = F' E + e
template <int S>
__device__ __forceinline__ void inv_round_a_derived(double (&x)[Sub<S>::E], const ArithF64 &ar,
                                                    const ulonglong2 *itw, const ulonglong2 *small, uint32_t base,
                                                    uint32_t F) {
    constexpr int LE = Sub<S>::LE, E = Sub<S>::E;
#pragma unroll
    for (int g = S - 1; g >= LE; g--) {
        const int d = 1 << (S - 1 - g);
        const ulonglong2 B = itw[(base << g) + (F << (LE - S + g))];
        ulonglong2 w[1 << (LE - 1)];
#pragma unroll
        for (int i = 0; i < (1 << (g + LE - S)); i++) w[i] = i == 0 ? B : ar.twmul(B, small[i]);
#pragma unroll
        for (int e = 0; e < E; e++) {
            if (e & d) continue;
            ar.gs(x[e], x[e + d], w[e >> (S - g)]);
        }
    }
}

// inverse, stages g = LE-1 .. 0 on u = F + T e (rows pass: never the last stage)
template <int S>
__device__ __forceinline__ void inv_round_b_derived(double (&x)[Sub<S>::E], const ArithF64 &ar,
                                                    const ulonglong2 *itw, const ulonglong2 *small, uint32_t base) {
    constexpr int LE = Sub<S>::LE, E = Sub<S>::E;
#pragma unroll
    for (int g = LE - 1; g >= 0; g--) {
        const int d = E >> (g + 1);
        const ulonglong2 B = itw[base << g];
        ulonglong2 w[1 << (LE - 1)];
#pragma unroll
        for (int i = 0; i < (1 << g); i++) w[i] = i == 0 ? B : ar.twmul(B, small[i]);
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
    static_assert(Sub<S2>::LE <= 5 && Sub<S1>::LE <= 5, "small twiddle table holds 16 entries");
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

template <class A, int S1, int S2>
__device__ __forceinline__ void fwd_cols_tile(const uint64_t (&raw)[Sub<S1>::E], const NttBatch &b,
                                              const NttTables &t, const TileRef &r, uint32_t prow, uint64_t q,
                                              typename A::T *lds) {
    using G = Geo<S1, S2>;
    using SB = Sub<S1>;
    using T = typename A::T;
    const A ar(q);
    const ulonglong2 *tw = t.tw + (size_t)prow * G::N;
    uint64_t *dst = b.dst + r.m * b.dstride + (size_t)r.l * G::N + r.tile * kCols;
    const uint32_t c = threadIdx.x % kCols, F = threadIdx.x / kCols;
    T x[SB::E];
#pragma unroll
    for (int e = 0; e < SB::E; e++) x[e] = ar.load(raw[e]);
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
#pragma unroll
    for (int e = 0; e < SB::E; e++) dst[(size_t)(F * SB::E + e) * G::N2 + c] = ar.store_mid(x[e]);
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
        for (int e = 0; e < SB::E; e++) raw[e] = s[(size_t)(F + SB::T * e) * G::N2 + c];
    }
    while (cur < total) {
        const uint32_t nxt = next_tile(b, G::COL_TILES, cur + gridDim.x, total);
        const TileRef r = decode_tile(b, G::COL_TILES, cur);
        uint64_t nraw[SB::E];
        if (nxt < total) {
            const uint64_t *s = cols_src<S1, S2>(b, decode_tile(b, G::COL_TILES, nxt), b.src, b.sstride);
#pragma unroll
            for (int e = 0; e < SB::E; e++) nraw[e] = s[(size_t)(F + SB::T * e) * G::N2 + c];
        }
        const uint32_t prow = b.map.row(r.l);
        const uint64_t q = t.mod[prow];
        if (q < kF64PrimeBound)
            fwd_cols_tile<ArithF64, S1, S2>(raw, b, t, r, prow, q, lds);
        else
            fwd_cols_tile<ArithInt, S1, S2>(raw, b, t, r, prow, q, reinterpret_cast<uint64_t *>(lds));
#pragma unroll
        for (int e = 0; e < SB::E; e++) raw[e] = nraw[e];
        cur = nxt;
        __syncthreads();
    }
}

// Rows pass: dst (intermediate) -> dst (canonical).
template <class A, int S1, int S2>
__device__ __forceinline__ void fwd_rows_tile(const uint64_t (&raw)[Sub<S2>::E], const NttBatch &b,
                                              const NttTables &t, const TileRef &r, uint32_t prow, uint64_t q,
                                              typename A::T *lds) {
    using G = Geo<S1, S2>;
    using SB = Sub<S2>;
    using T = typename A::T;
    const A ar(q);
    const ulonglong2 *tw = t.tw + (size_t)prow * G::N;
    const uint32_t F = threadIdx.x % SB::T, rr = threadIdx.x / SB::T;
    const uint32_t k1 = r.tile * G::ROWS + rr;
    uint64_t *rowp = b.dst + r.m * b.dstride + (size_t)r.l * G::N + (size_t)k1 * G::N2;
    T *lr = lds + rr * G::ROW_PITCH;
    T x[SB::E];
#pragma unroll
    for (int e = 0; e < SB::E; e++) x[e] = ar.load_mid(raw[e]);
    if constexpr (A::kF64)
        fwd_round_a_derived<S2>(x, ar, tw, t.small_fw + (size_t)prow * 16, G::N1 + k1);
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
        fwd_round_b_derived<S2>(x, ar, tw, t.small_fw + (size_t)prow * 16, G::N1 + k1, F);
    else
        fwd_round_b<A, S2>(x, ar, tw, G::N1 + k1, F);
    // transpose back through LDS so the stores are coalesced
    __syncthreads();
#pragma unroll
    for (int e = 0; e < SB::E; e++) lr[rpad(F * SB::E + e)] = x[e];
    __syncthreads();
#pragma unroll
    for (int e = 0; e < SB::E; e++) rowp[F + SB::T * e] = ar.store(lr[rpad(F + SB::T * e)]);
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
        for (int e = 0; e < SB::E; e++) raw[e] = s[F + SB::T * e];
    }
    while (cur < total) {
        const uint32_t nxt = next_tile(b, G::ROW_TILES, cur + gridDim.x, total);
        const TileRef r = decode_tile(b, G::ROW_TILES, cur);
        uint64_t nraw[SB::E];
        if (nxt < total) {
            const uint64_t *s = rows_ptr<S1, S2>(b, decode_tile(b, G::ROW_TILES, nxt), b.src, b.sstride);
#pragma unroll
            for (int e = 0; e < SB::E; e++) nraw[e] = s[F + SB::T * e];
        }
        const uint32_t prow = b.map.row(r.l);
        const uint64_t q = t.mod[prow];
        if (q < kF64PrimeBound)
            fwd_rows_tile<ArithF64, S1, S2>(raw, b, t, r, prow, q, lds);
        else
            fwd_rows_tile<ArithInt, S1, S2>(raw, b, t, r, prow, q, reinterpret_cast<uint64_t *>(lds));
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
                                              typename A::T *lds) {
    using G = Geo<S1, S2>;
    using SB = Sub<S2>;
    using T = typename A::T;
    const A ar(q);
    const ulonglong2 *itw = t.itw + (size_t)prow * G::N;
    const uint32_t F = threadIdx.x % SB::T, rr = threadIdx.x / SB::T;
    const uint32_t k1 = r.tile * G::ROWS + rr;
    uint64_t *drow = b.dst + r.m * b.dstride + (size_t)r.l * G::N + (size_t)k1 * G::N2;
    T *lr = lds + rr * G::ROW_PITCH;
    T x[SB::E];
#pragma unroll
    for (int e = 0; e < SB::E; e++) lr[rpad(F + SB::T * e)] = ar.load(raw[e]);
    __syncthreads();
#pragma unroll
    for (int e = 0; e < SB::E; e++) x[e] = lr[rpad(F * SB::E + e)];
    if constexpr (A::kF64)
        inv_round_a_derived<S2>(x, ar, itw, t.small_inv + (size_t)prow * 16, G::N1 + k1, F);
    else
        inv_round_a<A, S2>(x, ar, itw, G::N1 + k1, F);
    __syncthreads();
#pragma unroll
    for (int e = 0; e < SB::E; e++) lr[rpad(F * SB::E + e)] = x[e];
    __syncthreads();
#pragma unroll
    for (int e = 0; e < SB::E; e++) x[e] = lr[rpad(F + SB::T * e)];
    if constexpr (A::kF64)
        inv_round_b_derived<S2>(x, ar, itw, t.small_inv + (size_t)prow * 16, G::N1 + k1);
    else
        inv_round_b<A, S2, false>(x, ar, itw, G::N1 + k1, ulonglong2{0, 0});
#pragma unroll
    for (int e = 0; e < SB::E; e++) drow[F + SB::T * e] = ar.store_mid(x[e]);
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
        for (int e = 0; e < SB::E; e++) raw[e] = s[F + SB::T * e];
    }
    while (cur < total) {
        const uint32_t nxt = next_tile(b, G::ROW_TILES, cur + gridDim.x, total);
        const TileRef r = decode_tile(b, G::ROW_TILES, cur);
        uint64_t nraw[SB::E];
        if (nxt < total) {
            const uint64_t *s = rows_ptr<S1, S2>(b, decode_tile(b, G::ROW_TILES, nxt), b.src, b.sstride);
#pragma unroll
            for (int e = 0; e < SB::E; e++) nraw[e] = s[F + SB::T * e];
        }
        const uint32_t prow = b.map.row(r.l);
        const uint64_t q = t.mod[prow];
        if (q < kF64PrimeBound)
            inv_rows_tile<ArithF64, S1, S2>(raw, b, t, r, prow, q, lds);
        else
            inv_rows_tile<ArithInt, S1, S2>(raw, b, t, r, prow, q, reinterpret_cast<uint64_t *>(lds));
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
                                              typename A::T *lds) {
    using G = Geo<S1, S2>;
    using SB = Sub<S1>;
    using T = typename A::T;
    const A ar(q);
    const ulonglong2 *itw = t.itw + (size_t)prow * G::N;
    uint64_t *data = b.dst + r.m * b.dstride + (size_t)r.l * G::N + r.tile * kCols;
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
    for (int e = 0; e < SB::E; e++) data[(size_t)(F + SB::T * e) * G::N2 + c] = ar.store(x[e]);
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
        for (int e = 0; e < SB::E; e++) raw[e] = s[(size_t)(F * SB::E + e) * G::N2 + c];
    }
    while (cur < total) {
        const uint32_t nxt = next_tile(b, G::COL_TILES, cur + gridDim.x, total);
        const TileRef r = decode_tile(b, G::COL_TILES, cur);
        uint64_t nraw[SB::E];
        if (nxt < total) {
            const uint64_t *s = cols_src<S1, S2>(b, decode_tile(b, G::COL_TILES, nxt), b.src, b.sstride);
#pragma unroll
            for (int e = 0; e < SB::E; e++) nraw[e] = s[(size_t)(F * SB::E + e) * G::N2 + c];
        }
        const uint32_t prow = b.map.row(r.l);
        const uint64_t q = t.mod[prow];
        if (q < kF64PrimeBound)
            inv_cols_tile<ArithF64, S1, S2>(raw, b, t, r, prow, q, lds);
        else
            inv_cols_tile<ArithInt, S1, S2>(raw, b, t, r, prow, q, reinterpret_cast<uint64_t *>(lds));
#pragma unroll
        for (int e = 0; e < SB::E; e++) raw[e] = nraw[e];
        cur = nxt;
        __syncthreads();
    }
}

}  // namespace pfa
