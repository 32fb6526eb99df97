// Fused key-switching and rescale pipelines.
//
// The staged path (rns.hip) runs ModUp as INTT -> BConv -> NTT -> inner
// product, and ModDown / rescale as INTT -> BConv -> NTT -> epilogue, each a
// separate kernel with its result round-tripping through HBM.  Here the base
// conversion is computed inside the load stage of the forward NTT's columns
// pass, and the consumer of the forward NTT (the key-switch inner product, the
// ModDown epilogue, the rescale epilogue) runs inside its rows pass:
//
//   key switch c2 -> (cx0, cx1) over QlP:
//     1. INTT(c2) * [(Q_b/q_i)^-1]_{q_i}                       (ntt_inverse)
//     2. k_bconv_cols: per digit b and target limb r outside digit b,
//        y = sum_i t_i [Q_b/q_i]_{p_r} then the columns pass    -> I[b][r]
//     3. k_inner_ws: per target limb r, for every digit b: the rows pass
//        of I[b][r] (or c2 itself when r is in digit b), times key[b][k][r],
//        accumulated over b                                      -> cx[k][r]
//   ModDown cx -> out over Ql:
//     1. INTT(cx_P) * [(P/p_j)^-1]_{p_j}                        (ntt_inverse)
//     2. k_bconv_cols: y = sum_j xP_j [P/p_j]_{q_i}, columns pass -> D[m][i]
//     3. k_epi_rows: rows pass of D, out = base + (cx - D) [P^-1]_{q_i}
//   rescale c -> c' over Q_{l-1}:
//     1. INTT of the last limb                                  (ntt_inverse)
//     2. k_bconv_cols with one input limb and factor 1 (c_last mod q_j)
//     3. k_epi_rows: out = (c - D) [q_last^-1]_{q_j}
//
// Every step is the staged path's formula (the reference's: src/rns_bconv.cu
// :455-628 ModUp, src/eval_key_switch.cu:175-230 inner product,
// src/rns_bconv.cu:212-229 and include/ntt_radix8_tmpl.cuh:216-233 ModDown,
// src/rns.cu:1128-1158 rescale); only where the values live changes, and all
// outputs are canonical residues, so results are bit-identical.
//
// Base conversion in FP64 (target prime q < 2^50): the products t * m mod q
// use ArithF64::mulw with the matrix entry m as the constant.  An input residue
// t below 2^50 is exact in a double; a wider one (a 60-bit input prime) is
// split t = h 2^32 + l and converted as h [m 2^32]_q + l m.  Each product is
// within (-0.875 q, 0.875 q) (|t w / q| < 2^50, so fl(t wq) is within 3/8 of
// the true quotient); the sum is reduced whenever the next product could take
// it past 7 x 0.875 q, which keeps every partial sum below 2^53.  Targets q >= 2^50 use integer
// Shoup products, each in [0, 2q), summed with a conditional subtraction.
#include <algorithm>

#include "internal.h"
#include "ntt_kernels.h"

namespace pfa {

namespace {

// Rows per workgroup of the fused rows kernels: eight rows when that still
// makes a full wavefront, which doubles the number of work items against the
// NTT's rows pass (the inner-product kernel has only QlP x N1/ROWS items).
template <int S1, int S2>
struct FGeo {
    using G = Geo<S1, S2>;
    static constexpr int ROWS = Sub<S2>::T * 8 >= 64 ? 8 : G::ROWS;
    static constexpr int THREADS = ROWS * Sub<S2>::T;
    static constexpr int TILES = G::N1 / ROWS;
    static constexpr int LDS = ROWS * G::ROW_PITCH;
};

// ------------------------------------------------------------ base conversion
// One columns-pass job: target limb (table row prow) of one output poly, with
// inputs n_in limbs of `in` (limb stride N) over the table rows in_row0 + i.
struct BconvCols {
    const uint64_t *in;     // input limbs of group 0; group g adds g * in_gstride
    uint64_t *out;          // output limbs; job (g, j) writes out + g * out_gstride + j * N
    const ulonglong2 *bc;   // factor pairs [(m, m 2^32) in the target's policy]: see bc_of
    uint64_t in_gstride, out_gstride;
    // independent conversions of the same shape: member i adds i * in_bstride / out_bstride
    uint32_t batch = 1;
    uint64_t in_bstride = 0, out_bstride = 0;
    uint32_t groups;        // output polys (digits for ModUp, polys for ModDown / rescale)
    uint32_t J;             // target limbs per group (positions 0 .. J-1)
    uint32_t n_in;          // input limbs per group (<= alpha; the last ModUp digit may be short)
    uint32_t n_in_last;     // input limbs of the last group
    uint32_t in_row0;       // table row of input limb 0 of group 0
    uint32_t in_row_step;   // table rows between groups' first inputs (ModUp: alpha; else 0)
    // target position j -> table row: j < split ? j : split_base + (j - split)
    uint32_t split, split_base;
    // ModUp skips the group's own limbs: positions [g * skip_step, + n_in) are not written
    uint32_t skip;          // 1 for ModUp
    uint32_t bc_gstride;    // pairs between groups' factor blocks
    uint32_t bc_istride;    // pairs between one input's consecutive target factors... see bc_of
    // table row of input 0 when it differs from the run in_row0 + i (the fused
    // ModDown + rescale puts the rescale's last-limb coefficients first);
    // inputs i >= 1 then sit at rows in_row0 + i - 1.  ~0u: no such input
    uint32_t first_row = ~0u;
    // every factor is 1 (ModUp with alpha = 1: Q_b = q_i; the rescale's single
    // input): a lone input below 2^50 is then only reduced, not multiplied
    uint32_t unit = 0;
    // integer-policy targets with two inputs or more: 128-bit sums of the
    // inputs times the factors in Montgomery form (pair 1, m 2^64 mod q) and
    // one Montgomery reduction (the context's constants -q^-1 mod 2^64); set by
    // the launcher when every input sum stays below 2^64, else null (Shoup)
    const ulonglong2 *mont = nullptr;
    // position -> item table (a permutation of the launch's positions) built
    // for sched_grid workgroups over sched_total positions; the launcher drops
    // it when its launch differs.  null: position p runs item p
    const uint32_t *sched = nullptr;
    uint32_t sched_grid = 0, sched_total = 0;
};

__device__ __forceinline__ uint32_t bconv_in_row(const BconvCols &a, uint32_t row0, uint32_t i) {
    if (a.first_row == ~0u) return row0 + i;
    return i == 0 ? a.first_row : row0 + i - 1;
}

// factor pair index for (group g, input i, target j): bc[((g * n_in_max + i) * J + j) * 2 + h]
// (ModUp: per digit; ModDown / rescale: shared by all groups, bc_gstride = 0)
__device__ __forceinline__ const ulonglong2 *bc_of(const BconvCols &a, uint32_t g, uint32_t i, uint32_t j) {
    return a.bc + (size_t)g * a.bc_gstride + ((size_t)i * a.bc_istride + j) * 2;
}

template <class A, int S1, int S2>
__device__ __forceinline__ void bconv_source(const BconvCols &a, const NttTables &t, const A &ar, uint32_t mi,
                                             uint32_t g, uint32_t j, uint32_t tile, uint32_t prow,
                                             typename A::T (&x)[Sub<S1>::E]) {
    using G = Geo<S1, S2>;
    using SB = Sub<S1>;
    const uint32_t c = threadIdx.x % kCols, F = threadIdx.x / kCols;
    const uint32_t n_in = g + 1 == a.groups ? a.n_in_last : a.n_in;
    const uint64_t *base = a.in + (size_t)mi * a.in_bstride + (size_t)g * a.in_gstride + tile * kCols + c;
    const uint32_t row0 = a.in_row0 + g * a.in_row_step;
    if constexpr (A::kF64) {
        if (a.unit && n_in == 1 && t.mod[bconv_in_row(a, row0, 0)] < kF64PrimeBound) {
            // x = v mod q with v < 2^50: the FMA remainder of the nearest
            // quotient is exact and within (0.5 + 2^-20) q of zero
#pragma unroll
            for (int e = 0; e < SB::E; e++) {
                x[e] = ar.load(base[(size_t)(F + SB::T * e) * G::N2]);
                ar.reduce(x[e]);
            }
            return;
        }
        double acc[SB::E];
#pragma unroll
        for (int e = 0; e < SB::E; e++) acc[e] = 0.0;
        uint32_t units = 0;  // bound on |acc| in units of 0.875 q (a narrow product); kept <= 7
        for (uint32_t i = 0; i < n_in; i++) {
            const ulonglong2 *f = bc_of(a, g, i, j);
            const ulonglong2 f0 = f[0];
            const double w0 = ArithF64::as_f(f0.x), wq0 = ArithF64::as_f(f0.y);
            const uint64_t *src = base + (size_t)i * G::N;
            const bool wide = t.mod[bconv_in_row(a, row0, i)] >= kF64PrimeBound;
            if (units + (wide ? 2u : 1u) > 7u) {
#pragma unroll
                for (int e = 0; e < SB::E; e++) ar.reduce(acc[e]);
                units = 1;
            }
            units += wide ? 2u : 1u;
            if (wide) {
                const ulonglong2 f1 = f[1];
                const double w1 = ArithF64::as_f(f1.x), wq1 = ArithF64::as_f(f1.y);
#pragma unroll
                for (int e = 0; e < SB::E; e++) {
                    const uint64_t v = src[(size_t)(F + SB::T * e) * G::N2];
                    acc[e] += ar.mulw((double)(uint32_t)(v >> 32), w1, wq1) + ar.mulw((double)(uint32_t)v, w0, wq0);
                }
            } else {
#pragma unroll
                for (int e = 0; e < SB::E; e++) acc[e] += ar.mulw(ar.load(src[(size_t)(F + SB::T * e) * G::N2]), w0, wq0);
            }
        }
#pragma unroll
        for (int e = 0; e < SB::E; e++) {
            ar.reduce(acc[e]);
            x[e] = acc[e];
        }
    } else {
        const uint64_t q = ar.q, q2 = ar.q2;
        if (a.mont && n_in >= 2) {
            // sum_i t_i (m_i 2^64 mod q) < q sum_i t_i < q 2^64, so one
            // Montgomery reduction gives sum_i t_i m_i mod q in [0, 2q): 4
            // multiplies per input and 7 for the reduction, against a
            // 10-multiply Shoup product per input
            const uint64_t qn = ld_const(reinterpret_cast<const uint64_t *>(a.mont + prow));
            U128 acc[SB::E];
#pragma unroll
            for (int e = 0; e < SB::E; e++) acc[e] = U128{0, 0};
            for (uint32_t i = 0; i < n_in; i++) {
                const uint64_t mm = ld_const(reinterpret_cast<const uint64_t *>(bc_of(a, g, i, j) + 1));
                const uint64_t *src = base + (size_t)i * G::N;
#pragma unroll
                for (int e = 0; e < SB::E; e++) mac(acc[e], src[(size_t)(F + SB::T * e) * G::N2], mm);
            }
#pragma unroll
            for (int e = 0; e < SB::E; e++) x[e] = mont_reduce(acc[e], q, qn);
            return;
        }
        uint64_t acc[SB::E];
#pragma unroll
        for (int e = 0; e < SB::E; e++) acc[e] = 0;
        for (uint32_t i = 0; i < n_in; i++) {
            const ulonglong2 f0 = bc_of(a, g, i, j)[0];
            const uint64_t *src = base + (size_t)i * G::N;
#pragma unroll
            for (int e = 0; e < SB::E; e++)
                acc[e] = csub(acc[e] + shoup_lazy(src[(size_t)(F + SB::T * e) * G::N2], f0.x, f0.y, q), q2);
        }
#pragma unroll
        for (int e = 0; e < SB::E; e++) x[e] = acc[e];
    }
}

template <int S1, int S2>
__global__ void __launch_bounds__((Geo<S1, S2>::COL_THREADS)) k_bconv_cols(BconvCols a, NttTables t) {
    using G = Geo<S1, S2>;
    using SB = Sub<S1>;
    __shared__ double lds[G::COL_LDS];
    __shared__ ulonglong2 twl[G::N1];  // the target prime's columns-pass twiddles
    const uint32_t NG = a.batch * a.groups * G::COL_TILES;
    const uint32_t total = grouped_total(NG, a.J);
    for (uint32_t p = blockIdx.x; p < total; p += gridDim.x) {
        const uint32_t w = a.sched ? ld_const(a.sched + p) : p;
        uint32_t gt, j;
        if (!grouped_item(w, NG, a.J, gt, j)) continue;
        const uint32_t mg = gt / G::COL_TILES, tile = gt % G::COL_TILES;
        const uint32_t mi = mg / a.groups, g = mg % a.groups;
        if (a.skip && j >= g * a.n_in && j < g * a.n_in + (g + 1 == a.groups ? a.n_in_last : a.n_in)) continue;
        const uint32_t prow = j < a.split ? j : a.split_base + (j - a.split);
        const uint64_t q = t.mod[prow];
        uint64_t *olimb = a.out + (size_t)mi * a.out_bstride + (size_t)g * a.out_gstride + (size_t)j * G::N;
        // the twiddles are requested before the inputs and staged in LDS
        TwStage<G::N1, G::COL_THREADS> st;
        st.load([&](uint32_t i) { return t.tw[(size_t)prow * G::N + i]; });
        if (q < kF64PrimeBound) {
            const ArithF64 ar(q);
            double x[SB::E];
            bconv_source<ArithF64, S1, S2>(a, t, ar, mi, g, j, tile, prow, x);
            st.store(twl);
            __syncthreads();
            fwd_cols_core<ArithF64, S1, S2>(x, ar, twl, lds);
            fwd_cols_store<ArithF64, S1, S2>(x, ar, tile, olimb);
        } else {
            const ArithInt ar(q);
            uint64_t x[SB::E];
            bconv_source<ArithInt, S1, S2>(a, t, ar, mi, g, j, tile, prow, x);
            st.store(twl);
            __syncthreads();
            fwd_cols_core<ArithInt, S1, S2>(x, ar, twl, reinterpret_cast<uint64_t *>(lds));
            fwd_cols_store<ArithInt, S1, S2>(x, ar, tile, olimb);
        }
        __syncthreads();
    }
}

// ------------------------------------------------------------ inner product
struct InnerRows {
    const uint64_t *inter;  // [beta][QlP][N] columns-pass output of the base conversion
    const uint64_t *c2;     // [Ql][N] NTT form: the digit's own limbs
    const uint64_t *key;    // [dnum][2][QP][N] (member i: key_table[i] when key_table is set)
    uint64_t *cx;           // [2][QlP][N]
    const ulonglong2 *mont;  // [QP] Montgomery constants (-q^-1 mod 2^64, 2^128 mod q)
    uint32_t Ql, QlP, alpha, beta, Q, QP;
    // independent key switches with the same key: member i adds i * the stride
    uint32_t batch = 1;
    uint64_t inter_bstride = 0, c2_bstride = 0, cx_bstride = 0;
    // ModDown + rescale fusion (batch 1 only): output k of target limb fold_r
    // (the level's last prime) is written as base_k[fold_r] + acc * fold_f,
    // fold_f = [P^-1]_q as an integer Shoup pair; ~0u = no folding
    uint32_t fold_r = ~0u;
    const uint64_t *fold_base0 = nullptr, *fold_base1 = nullptr;
    uint64_t fold_bstride = 0;  // member i's bases at + i fold_bstride
    const ulonglong2 *fold_f = nullptr;
    // Items from `full` on are split by digit range (see k_inner_ws): rem
    // items of kch chunks each; chunk c of item full + j writes its canonical
    // sums to partial + (j kch + c) 2 ROWS N2, and the last chunk of the item to
    // arrive (counter[j]) adds them and writes the output.
    uint32_t full = ~0u;
    uint32_t rem = 0, kch = 1;
    uint64_t *partial = nullptr;
    uint32_t *counter = nullptr;
    uint32_t *host_err = nullptr;  // mapped pinned host word: error bit 4 is stored there
    const uint64_t *const *key_table = nullptr;  // per-member keys (device array), or null
    uint32_t member_fast = 0;  // item order: member index fastest (see ws_decode)
    // target of item group i: order[i] (null: i).  Items of integer-policy
    // targets take ~1.5-2.25x as long as FP64 ones; ordered last, they are the
    // first to be split when items are left over after whole rounds.
    const uint32_t *order = nullptr;
};

__device__ __forceinline__ uint32_t ws_target(const InnerRows &a, uint32_t i) { return a.order ? a.order[i] : i; }

// Item w0 -> (member mi, item w of that member).  With several members the
// members' items of one (target, tile) read the same key rows (one key for the
// batch): they are given workgroups congruent mod 8, which run on one XCD
// (workgroups are dealt to the XCDs round-robin), so the rows come from HBM
// once and are shared through that XCD's L2 (the grouped order of
// grouped_item, with the members as the group's items; needs a multiple of 8
// items per member, else the members only run fastest).
__device__ __forceinline__ void ws_decode(const InnerRows &a, uint32_t w0, uint32_t tiles, uint32_t &mi,
                                         uint32_t &w) {
    const uint32_t per = a.QlP * tiles;
    if (a.member_fast && per % kXcds == 0) {
        grouped_item(w0, per, a.batch, w, mi);
    } else if (a.member_fast) {
        mi = w0 % a.batch;
        w = w0 / a.batch;
    } else {
        mi = w0 / per;
        w = w0 % per;
    }
}

// Digit b's input for limb r at row offset rowoff: the digit's own limb of c2
// (already in NTT form) or the columns-pass output to transform.
__device__ __forceinline__ const uint64_t *inner_src(const InnerRows &a, uint32_t b, uint32_t r, size_t rowoff,
                                                     uint32_t N, bool &own) {
    own = r < a.Ql && r >= b * a.alpha && r < b * a.alpha + a.alpha;
    // chosen by arithmetic: a select between the two pointers made the compiler
    // keep them in a scratch array, whose per-digit load (a vector memory
    // access) waited behind the prefetched tile
    const uintptr_t c2p = (uintptr_t)(a.c2 + (size_t)r * N + rowoff);
    const uintptr_t inp = (uintptr_t)(a.inter + ((size_t)b * a.QlP + r) * N + rowoff);
    return (const uint64_t *)(inp + (uintptr_t)own * (c2p - inp));
}

// One work item is a (target limb r, tile of ROWS rows) pair; its digits are
// processed in turn by a warp-specialized workgroup.  The first half of the
// workgroup (the transform waves) runs digit b's rows pass into one of two LDS
// buffers while the second half (the accumulate waves) multiplies digit b-1's
// transformed tile, read from the other buffer, by its key limbs.  The roles
// keep disjoint register state (transform: the tile and the next digit's
// prefetched tile; accumulate: the accumulators and the next digit's key
// limbs), so the key traffic overlaps the transforms of the other waves.
// A row's threads are all in one wave, so the rows pass exchanges data within
// each wave only (wave_lds_sync) and the roles meet at one workgroup barrier
// per digit, the hand-off of the buffers; between two barriers both roles work.
// With two accumulate waves or more, each takes one output (0 or 1) of the
// whole tile, AE elements per thread, in the order the key is laid out.
//
// Two properties keep the prefetches a full step ahead:
// * Global loads complete in issue order (one vmcnt counter), so a load issued
//   after a prefetch cannot be waited for without waiting for the prefetch.
//   The FP64 rows-pass twiddle factors therefore come from LDS: the item's
//   rows' base factors and the small table are staged there once per item.
//   The Montgomery constants are loaded before the first key limbs.
// * Every prefetch is unconditional (the step after the last one reloads the
//   rows it has just consumed, which are still in L2), so the prefetched
//   registers are never merged with their previous values at the loop head,
//   which would cost a copy of each and ~60 registers.
template <int S1, int S2>
struct WsGeo {
    using G = Geo<S1, S2>;
    static constexpr int ROWS = FGeo<S1, S2>::ROWS;
    static constexpr int HALF = ROWS * Sub<S2>::T;  // threads per role
    static constexpr int THREADS = 2 * HALF;
    static constexpr int TILES = G::N1 / ROWS;
    static constexpr int LDS = 2 * ROWS * G::ROW_PITCH;      // doubles: the two tile buffers
    static constexpr int TW_RB = S2 * ROWS;                   // staged base factors [S2][ROWS]
    static constexpr int TW_SMALL = 1 << (S2 - 1);            // staged small table entries
    static constexpr int TW = TW_RB + TW_SMALL;               // ulonglong2 entries after the buffers
    // FP64 policy: the item's rows' twiddle values, one row of 2^S2 - 1 per
    // tile row (doubles after the staged entries), built once per item; up to
    // N2 = 256, where the table (16 KiB) still leaves 3 workgroups per CU
    static constexpr bool USE_TAB = S2 <= 8;
    static constexpr int TAB_ROW = G::N2 - 1;
    static constexpr int TAB = USE_TAB ? ROWS * TAB_ROW : 0;
    static_assert(!USE_TAB || 2 * TW <= ROWS * G::ROW_PITCH, "staged entries must fit in one tile buffer");
    // accumulate role: outputs per thread, threads per output, elements per thread and output
    static constexpr int NO = HALF >= 128 ? 1 : 2;
    static constexpr int TPO = NO == 1 ? HALF / 2 : HALF;
    static constexpr int AE = ROWS * G::N2 / TPO;
    static_assert(HALF % 64 == 0, "each role must be whole wavefronts");
    static_assert(TPO % 64 == 0 && ROWS * G::N2 % TPO == 0, "each output must be whole wavefronts");
};

// Orders this wave's LDS accesses around an exchange between its lanes: a
// wave's LDS operations execute in issue order, so the exchange needs no
// workgroup barrier, only that the compiler keep the accesses in order.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <class A, int S1, int S2>
__device__ __forceinline__ void ws_transform(const InnerRows &a, const NttTables &t, const A &ar, uint32_t r,
                                             uint32_t prow, uint32_t k1, uint32_t rr, const ulonglong2 *tws,
                                             const double *tab, typename A::T *b0, typename A::T *b1, uint32_t db,
                                             uint32_t de) {
    using G = Geo<S1, S2>;
    using W = WsGeo<S1, S2>;
    using SB = Sub<S2>;
    using T = typename A::T;
    const uint32_t F = (threadIdx.x % W::HALF) % SB::T;
    const size_t rowoff = (size_t)k1 * G::N2 + F;
    uint64_t nraw[SB::E];
    bool nown;
    {
        const uint64_t *s = inner_src(a, db, r, rowoff, G::N, nown);
#pragma unroll
        for (int e = 0; e < SB::E; e++) nraw[e] = ld_stream(&s[SB::T * e]);
    }
    for (uint32_t b = db; b < de; b++) {
        T *buf = ((b - db) & 1u) ? b1 : b0;
        const bool own = nown;
        T x[SB::E];
#pragma unroll
        for (int e = 0; e < SB::E; e++) x[e] = own ? ar.load(nraw[e]) : ar.load_mid(nraw[e]);
        {
            const uint64_t *s = inner_src(a, b + 1 < de ? b + 1 : b, r, rowoff, G::N, nown);
#pragma unroll
            for (int e = 0; e < SB::E; e++) nraw[e] = ld_stream(&s[SB::T * e]);
        }
        if (!own) {
            // the twiddle addresses are made opaque per digit: left loop-invariant,
            // the compiler would hold every twiddle live across the digit loop
            if constexpr (A::kF64 && W::USE_TAB) {
                uint32_t kr = rr;
                asm volatile("" : "+v"(kr));
                fwd_round_a_tab<S2>(x, ar, tab + kr * W::TAB_ROW);
            } else if constexpr (A::kF64) {
                uint32_t kr = rr;
                asm volatile("" : "+v"(kr));
                fwd_round_a_derived<S2, W::ROWS>(x, ar, tws, tws + W::TW_RB, kr);
            } else {
                uint32_t kr = k1, pr = prow;
                asm volatile("" : "+v"(kr), "+s"(pr));
                fwd_round_a<A, S2>(x, ar, t.tw + (size_t)pr * G::N, G::N1 + kr);
            }
#pragma unroll
            for (int e = 0; e < SB::E; e++) ar.reduce(x[e]);
#pragma unroll
            for (int e = 0; e < SB::E; e++) buf[rpad(F + SB::T * e)] = x[e];
            wave_lds_sync();
#pragma unroll
            for (int e = 0; e < SB::E; e++) x[e] = buf[rpad(F * SB::E + e)];
            if constexpr (A::kF64 && W::USE_TAB) {
                uint32_t kr = rr;
                asm volatile("" : "+v"(kr));
                fwd_round_b_tab<S2>(x, ar, tab + kr * W::TAB_ROW, F);
            } else if constexpr (A::kF64) {
                uint32_t kr = rr;
                asm volatile("" : "+v"(kr));
                fwd_round_b_derived<S2, W::ROWS>(x, ar, tws, tws + W::TW_RB, kr, F);
            } else {
                uint32_t kr = k1, pr = prow;
                asm volatile("" : "+v"(kr), "+s"(pr));
                fwd_round_b<A, S2>(x, ar, t.tw + (size_t)pr * G::N, G::N1 + kr, F);
            }
            wave_lds_sync();
#pragma unroll
            for (int e = 0; e < SB::E; e++) buf[rpad(F * SB::E + e)] = x[e];
        } else {
#pragma unroll
            for (int e = 0; e < SB::E; e++) buf[rpad(F + SB::T * e)] = x[e];
        }
        __syncthreads();  // buffer (b - db) % 2 to the accumulate waves
    }
    __syncthreads();  // the accumulate waves consume the last digit
}

// Product of digit d's transformed element x (lazy) with key limb value w,
// accumulated into acc: FP64 policy exact products (acc reduced every second
// digit); integer policy Montgomery products x w 2^-64, each in [0, 2q), summed
// in [0, 2q) (ws_sum turns the sum back into sum x w mod q).
template <class A>
__device__ __forceinline__ void ws_mac(const A &ar, typename A::T &acc, typename A::T x, uint64_t w, ulonglong2 mt) {
    if constexpr (A::kF64) {
        ar.reduce(x);
        const double wd = ar.load(w);
        acc += ar.mulw(x, wd, wd * ar.qinv);
    } else {
        acc = csub(acc + mont_mul(x, w, ar.q, mt.x), ar.q2);
    }
}

// The canonical residue of an accumulated sum.
template <class A>
__device__ __forceinline__ uint64_t ws_sum(const A &ar, typename A::T acc, ulonglong2 mt) {
    if constexpr (A::kF64)
        return ar.store(acc);
    else
        return ar.store(mont_mul(acc, mt.y, ar.q, mt.x));  // (sum 2^-64) 2^128 2^-64
}

// Output k of limb r at offset off (within the limb): the canonical sum v, or
// with the fold (see InnerRows) base_k + v [P^-1]_q.
__device__ __forceinline__ void ws_out(const InnerRows &a, uint32_t k, uint32_t r, size_t off, uint32_t N,
                                       uint64_t q, uint64_t v) {
    if (r == a.fold_r) {
        const ulonglong2 f = *a.fold_f;
        // base k as pointer arithmetic: a select between the two pointers made
        // the compiler keep them in a scratch array indexed by k
        const uintptr_t b0 = (uintptr_t)a.fold_base0, b1 = (uintptr_t)a.fold_base1;
        const uint64_t *fb = (const uint64_t *)(b0 + (uintptr_t)k * (b1 - b0));
        v = add_mod(shoup(v, f.x, f.y, q), fb[(size_t)r * N + off], q);
    }
    st_stream(a.cx + ((size_t)k * a.QlP + r) * N + off, v);
}

// Accumulates digits db .. de-1 of the tile (B0 / B1: the two tile buffers);
// with part null the item is whole and its output is written, else the
// canonical sums go to part ([2][ROWS][N2]).
template <class A, int S1, int S2>
__device__ __forceinline__ void ws_accumulate(const InnerRows &a, const A &ar, uint32_t r, uint32_t prow,
                                              uint32_t tile, const typename A::T *B0, const typename A::T *B1,
                                              uint32_t db, uint32_t de, uint64_t *part) {
    using G = Geo<S1, S2>;
    using W = WsGeo<S1, S2>;
    using T = typename A::T;
    constexpr int NO = W::NO, AE = W::AE, TPO = W::TPO;
    const uint32_t u = threadIdx.x - W::HALF;
    const uint32_t lane = u % TPO, kf = NO == 1 ? u / TPO : 0;  // kf: this thread's output when NO == 1
    const size_t tbase = (size_t)tile * W::ROWS * G::N2 + lane;  // element offset within a limb
    const size_t keyrow = (size_t)prow * G::N + tbase;
    const uint64_t QPN = (uint64_t)a.QP * G::N;
    // limb i = 2 d + k of the key (digit d, output k) at this thread's positions
    auto key_at = [&](uint32_t i) { return a.key + (size_t)i * QPN + keyrow; };
    ulonglong2 mt = a.mont[prow];
    mt.x = wave_uniform(mt.x);
    mt.y = wave_uniform(mt.y);
    __builtin_amdgcn_sched_barrier(0);
    T acc[NO][AE];
    uint64_t kw[NO][AE];
#pragma unroll
    for (int o = 0; o < NO; o++) {
        const uint64_t *k = key_at(2 * db + (NO == 1 ? kf : o));
#pragma unroll
        for (int i = 0; i < AE; i++) {
            acc[o][i] = 0;
            kw[o][i] = k[(size_t)TPO * i];
        }
    }
    __syncthreads();  // step 0: the transform waves fill buffer 0
    // Step s consumes digit d = db + s - 1; its key limbs were requested a whole
    // step earlier.  Key limbs use plain loads (unlike the streamed residues): a
    // key is reused call after call (relinearization, a rotation step repeated).
    for (uint32_t st = 1; st <= de - db; st++) {
        const uint32_t d = db + st - 1;
        const T *buf = ((st - 1) & 1u) ? B1 : B0;
#pragma unroll
        for (int i = 0; i < AE; i++) {
            const uint32_t p = lane + (uint32_t)TPO * i;
            const T x = buf[(p / G::N2) * G::ROW_PITCH + rpad(p % G::N2)];
#pragma unroll
            for (int o = 0; o < NO; o++) {
                ws_mac(ar, acc[o][i], x, kw[o][i], mt);
                if constexpr (!A::kF64) __builtin_amdgcn_sched_barrier(0);  // one integer product at a time
            }
        }
        // keep the refill after the products so it can reuse their key registers
        __builtin_amdgcn_sched_barrier(0);
        {
            // after the last digit: reload the limbs just consumed (still in L2)
            const uint32_t dn = d + 1 < de ? d + 1 : d;
#pragma unroll
            for (int o = 0; o < NO; o++) {
                const uint64_t *k = key_at(2 * dn + (NO == 1 ? kf : o));
#pragma unroll
                for (int i = 0; i < AE; i++) kw[o][i] = k[(size_t)TPO * i];
            }
        }
        if constexpr (A::kF64) {
            if (!(st & 1u)) {
#pragma unroll
                for (int o = 0; o < NO; o++)
#pragma unroll
                    for (int i = 0; i < AE; i++) ar.reduce(acc[o][i]);
            }
        }
        __syncthreads();
    }
    if (part) {
        // a digit chunk: plain stores, so the sums stay in the XCD's L2 for the
        // chunk that adds them
#pragma unroll
        for (int o = 0; o < NO; o++) {
            uint64_t *pk = part + (size_t)(NO == 1 ? kf : o) * W::ROWS * G::N2 + lane;
#pragma unroll
            for (int i = 0; i < AE; i++) pk[(size_t)TPO * i] = ws_sum(ar, acc[o][i], mt);
        }
        return;
    }
    const uint64_t q = (uint64_t)ar.q;
#pragma unroll
    for (int o = 0; o < NO; o++)
#pragma unroll
        for (int i = 0; i < AE; i++)
            ws_out(a, NO == 1 ? kf : o, r, tbase + (size_t)TPO * i, G::N, q, ws_sum(ar, acc[o][i], mt));
}

// One work item (target limb r of member mi, a tile of ROWS rows) over digits
// db .. de-1.
template <int S1, int S2>
__device__ __forceinline__ void ws_item(const InnerRows &a0, const NttTables &t, uint32_t w0, uint32_t db,
                                        uint32_t de, uint64_t *part, double *lds, ulonglong2 *tws) {
    using G = Geo<S1, S2>;
    using W = WsGeo<S1, S2>;
    double *tab = lds + W::LDS;
    const bool transform = threadIdx.x < W::HALF;
    const uint32_t rr = (threadIdx.x % W::HALF) / Sub<S2>::T;
    uint32_t mi, w;
    ws_decode(a0, w0, W::TILES, mi, w);
    InnerRows a = a0;
    a.inter += mi * a0.inter_bstride;
    a.c2 += mi * a0.c2_bstride;
    a.cx += mi * a0.cx_bstride;
    if (a0.key_table)  // member mi's key, a scalar load (mi is uniform)
        a.key = reinterpret_cast<const uint64_t *>(
            wave_uniform(ld_const(reinterpret_cast<const uint64_t *>(a0.key_table + mi))));
    {
        // member mi's fold bases (stride 0 without a batched fold); the offset
        // is made explicitly wave-uniform for the compiler
        const uint64_t fo = wave_uniform((uint64_t)mi * a0.fold_bstride);
        a.fold_base0 += fo;
        a.fold_base1 += fo;
    }
    const uint32_t r = ws_target(a, w / W::TILES), tile = w % W::TILES;
    const uint32_t prow = r < a.Ql ? r : a.Q + (r - a.Ql);
    const uint64_t q = wave_uniform(t.mod[prow]);
    const uint32_t k1 = tile * W::ROWS + rr;
    if (q < kF64PrimeBound) {
        double *b0 = lds + rr * G::ROW_PITCH, *b1 = b0 + W::ROWS * G::ROW_PITCH;
        if (transform) {
            // this item's rows' base factors rb[g][tile ROWS + i] and the small table
            const ulonglong2 *rb = t.rb_fw + (size_t)prow * S2 * G::N1 + tile * W::ROWS;
            const ulonglong2 *small = t.small_fw + (size_t)prow * kSmall;
            for (uint32_t i = threadIdx.x; i < (uint32_t)W::TW; i += W::HALF)
                tws[i] = i < (uint32_t)W::TW_RB ? rb[(i / W::ROWS) * G::N1 + i % W::ROWS] : small[i - W::TW_RB];
        }
        __syncthreads();
        // the rows' twiddle values once per item (they do not depend on the
        // digit): each digit's rows pass then reads them instead of deriving
        // them, which shortens the transform role, the longer of the two
        if constexpr (W::USE_TAB) {
            build_row_tab<S2, W::ROWS>(tab, ArithF64(q), tws, tws + W::TW_RB, threadIdx.x, W::THREADS);
            __syncthreads();
        }
        if (transform)
            ws_transform<ArithF64, S1, S2>(a, t, ArithF64(q), r, prow, k1, rr, tws, tab, b0, b1, db, de);
        else
            ws_accumulate<ArithF64, S1, S2>(a, ArithF64(q), r, prow, tile, lds, lds + W::ROWS * G::ROW_PITCH, db, de,
                                             part);
    } else {
        uint64_t *b0 = reinterpret_cast<uint64_t *>(lds) + rr * G::ROW_PITCH, *b1 = b0 + W::ROWS * G::ROW_PITCH;
        if (transform)
            ws_transform<ArithInt, S1, S2>(a, t, ArithInt(q), r, prow, k1, rr, tws, tab, b0, b1, db, de);
        else
            ws_accumulate<ArithInt, S1, S2>(a, ArithInt(q), r, prow, tile, reinterpret_cast<uint64_t *>(lds),
                                             reinterpret_cast<uint64_t *>(lds) + W::ROWS * G::ROW_PITCH, db, de, part);
    }
}

// The last chunk of split item w0 to finish adds the kch partial sums
// (canonical, in this XCD's L2) and writes the output.
template <int S1, int S2>
__device__ __forceinline__ void ws_combine(const InnerRows &a0, const NttTables &t, uint32_t w0,
                                           const uint64_t *parts) {
    using G = Geo<S1, S2>;
    using W = WsGeo<S1, S2>;
    using SB = Sub<S2>;
    const uint32_t F = (threadIdx.x % W::HALF) % SB::T, rr = (threadIdx.x % W::HALF) / SB::T;
    uint32_t mi, w;
    ws_decode(a0, w0, W::TILES, mi, w);
    InnerRows a = a0;
    a.cx += mi * a0.cx_bstride;
    {
        // member mi's fold bases (stride 0 without a batched fold); the offset
        // is made explicitly wave-uniform for the compiler
        const uint64_t fo = wave_uniform((uint64_t)mi * a0.fold_bstride);
        a.fold_base0 += fo;
        a.fold_base1 += fo;
    }
    const uint32_t r = ws_target(a, w / W::TILES), tile = w % W::TILES;
    const uint32_t prow = r < a.Ql ? r : a.Q + (r - a.Ql);
    const uint64_t q = wave_uniform(t.mod[prow]);
    const size_t rowoff = (size_t)(tile * W::ROWS + rr) * G::N2 + F;
    constexpr size_t PS = (size_t)2 * W::ROWS * G::N2;  // one chunk's sums
    const uint64_t *p = parts + (size_t)rr * G::N2 + F;
    uint64_t v0[SB::E], v1[SB::E];
#pragma unroll
    for (int e = 0; e < SB::E; e++) v0[e] = v1[e] = 0;
    // one chunk at a time, its 2 E loads in flight together
    for (uint32_t c = 0; c < a.kch; c++) {
        uint64_t l0[SB::E], l1[SB::E];
#pragma unroll
        for (int e = 0; e < SB::E; e++) {
            l0[e] = p[c * PS + SB::T * e];
            l1[e] = p[c * PS + (size_t)W::ROWS * G::N2 + SB::T * e];
        }
#pragma unroll
        for (int e = 0; e < SB::E; e++) {
            v0[e] = add_mod(v0[e], l0[e], q);
            v1[e] = add_mod(v1[e], l1[e], q);
        }
    }
#pragma unroll
    for (int e = 0; e < SB::E; e++) {
        ws_out(a, 0, r, rowoff + SB::T * e, G::N, q, v0[e]);
        ws_out(a, 1, r, rowoff + SB::T * e, G::N, q, v1[e]);
    }
}

// Items 0 .. full-1 are processed whole, item full - 1 - i by workgroup
// i mod grid.  When the item count is not a multiple of the resident
// workgroups, the rem items left over would run as a second round on a mostly
// idle chip; they are split into kch digit chunks instead, which fill one
// short round.  Counting workgroups from the end of the grid,
// g = grid - 1 - blockIdx, workgroup g takes chunk (u mod kch) of item
// full + (u / kch) 8 + (g mod 8), u = g / 8.  Both directions hand the last
// items to the workgroups dispatched first: with one member those are the
// integer-policy targets, the longest items.  Interleaved on one box against
// the forward directions: config 3 HMult 263.5 -> 255.7 us, L = 35
// 781.3 -> 747.5 us, batch-1 rotation 189.2 -> 184.2 us (the reversed chunks
// alone: L = 35 -4.3 to -4.5% on two boxes; the reversed whole items alone:
// config 3 -3%, rotation -3%; in separate processes BSGS 27.0 -> 26.4-26.7 ms,
// bootstrap 28.5 -> 28.2-28.3 ms), the same residues.  The grid is a multiple of
// 8, so the chunks of an item run on workgroups congruent mod 8, i.e. on one XCD (a
// launch's workgroups are dealt to the 8 XCDs round-robin), and their partial
// sums meet in that XCD's L2; nothing waits for anything.  Each chunk marks
// its XCD in the item's counter, and the last to arrive records an error if
// they differ.
//
// At N = 2^16 the kernel is compiled for 3 waves per SIMD (168 VGPRs): the
// integer-policy accumulate path would take 176, and the values the compiler
// then spills are loop invariants reloaded once per item (measured: L = 35
// inner product 540 -> 520 us against 2 waves per SIMD).
template <int S1, int S2>
struct WsWaves {
    static constexpr int MIN = S1 == 8 && S2 == 8 ? 3 : 1;
};

template <int S1, int S2>
__global__ void __launch_bounds__((WsGeo<S1, S2>::THREADS)) __attribute__((amdgpu_waves_per_eu(WsWaves<S1, S2>::MIN, 8)))
k_inner_ws(InnerRows a0, NttTables t) {
    using W = WsGeo<S1, S2>;
    // with the table, the staged entries (needed only to build it) live in
    // the second tile buffer, which the first digit leaves unused
    __shared__ double lds[W::LDS + (W::USE_TAB ? 0 : 2 * W::TW) + W::TAB];
    __shared__ uint32_t s_last;
    ulonglong2 *tws = reinterpret_cast<ulonglong2 *>(lds + (W::USE_TAB ? W::ROWS * Geo<S1, S2>::ROW_PITCH : W::LDS));
    const uint32_t total = a0.batch * a0.QlP * W::TILES;
    const uint32_t full = a0.full < total ? a0.full : total;
    for (uint32_t i = blockIdx.x; i < full; i += gridDim.x) {
        const uint32_t w0 = full - 1 - i;  // the last items (the longest) first
        ws_item<S1, S2>(a0, t, w0, 0, a0.beta, nullptr, lds, tws);
        __syncthreads();
    }
    if (a0.rem == 0) return;
    const uint32_t g = gridDim.x - 1 - blockIdx.x;
    const uint32_t u = g / kXcds, c = u % a0.kch;
    const uint32_t j = (u / a0.kch) * kXcds + g % kXcds;
    if (j >= a0.rem) return;
    constexpr size_t PS = (size_t)2 * W::ROWS * Geo<S1, S2>::N2;
    const uint64_t *parts = a0.partial + (size_t)j * a0.kch * PS;
    ws_item<S1, S2>(a0, t, full + j, c * a0.beta / a0.kch, (c + 1) * a0.beta / a0.kch,
                    a0.partial + ((size_t)j * a0.kch + c) * PS, lds, tws);
    // the chunk's sums are in L2 before its arrival is counted
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t mine = 1u << (8 + (xcc_id() & (kXcds - 1)));
        uint32_t *cnt = a0.counter + j;
        __hip_atomic_fetch_or(cnt, mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint32_t old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const bool last = (old & 0xffu) == a0.kch - 1;
        if (last) {
            if (((old | mine) & ~0xffu) != mine) {
                __hip_atomic_store(a0.host_err, 4u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            }
            __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // ready for the next launch
        }
        s_last = last ? 1u : 0u;
    }
    __syncthreads();
    if (s_last && threadIdx.x >= W::HALF) {
        asm volatile("buffer_inv sc0" ::: "memory");  // the other chunks' sums: read L2, not this CU's L1
        ws_combine<S1, S2>(a0, t, full + j, parts);
    }
}

// ------------------------------------------------------------ epilogue rows
// out[m][j] = (base[m][j] if given) + (c[m][j] - NTT(D[m][j])) f_j   (mod q_j)
struct EpiRows {
    const uint64_t *inter;  // [M][J][N] columns-pass output
    const uint64_t *c;      // [M][..][N], poly stride c_stride
    const uint64_t *base0, *base1;  // [J][N] each, or null: polys 2i and 2i+1 add base0/base1 + i base_stride
    uint64_t *out;          // [M][J][N]
    const ulonglong2 *f;    // [J] pairs in each limb's NTT policy
    uint64_t c_stride;
    uint32_t M, J;
    uint64_t base_stride = 0;
    // fused ModDown + rescale: when set ([J] pairs in each limb's NTT policy),
    // out = (c f1 + base - NTT(D)) f instead
    const ulonglong2 *f1 = nullptr;
    // the launcher may look up (and on first use build) a work schedule; the
    // allocation-free rescale turns that off
    bool allow_sched = true;
    // position -> item table for sched_grid workgroups over sched_total
    // positions (set by the launcher), or null: position p runs item p
    const uint32_t *sched = nullptr;
    uint32_t sched_grid = 0, sched_total = 0;
};

template <class A, int S1, int S2>
__device__ __forceinline__ void epi_item(const EpiRows &a, const NttTables &t, const A &ar, uint32_t m, uint32_t j,
                                         uint32_t k1, typename A::T *lr, ulonglong2 *twl) {
    using G = Geo<S1, S2>;
    using SB = Sub<S2>;
    using T = typename A::T;
    const uint32_t F = threadIdx.x % SB::T;
    const size_t rowoff = (size_t)k1 * G::N2 + F;
    const size_t lo = ((size_t)m * a.J + j) * G::N + rowoff;
    T x[SB::E];
#pragma unroll
    for (int e = 0; e < SB::E; e++) x[e] = ar.load_mid(ld_stream(&a.inter[lo + SB::T * e]));
    if constexpr (A::kF64) {
        // stage this item's rows' base factors rb[g][tile ROWS + i] and the
        // small table in LDS (requested after the residues, so the one wait
        // covers both) instead of dependent global reads inside the rounds
        using FG = FGeo<S1, S2>;
        constexpr int RB = S2 * FG::ROWS, NS = RB + (1 << (S2 - 1));
        const uint32_t tile0 = k1 - k1 % FG::ROWS;
        const ulonglong2 *rb = t.rb_fw + (size_t)j * S2 * G::N1 + tile0;
        const ulonglong2 *small = t.small_fw + (size_t)j * kSmall;
        TwStage<NS, FG::THREADS> st;
        st.load([&](uint32_t i) { return i < (uint32_t)RB ? rb[(i / FG::ROWS) * G::N1 + i % FG::ROWS] : small[i - RB]; });
        st.store(twl);
        __syncthreads();
        const TileTw w{nullptr, nullptr, twl, twl + RB, k1 % FG::ROWS};
        fwd_rows_core<A, S1, S2, FG::ROWS>(x, ar, w, k1, lr);
    } else {
        fwd_rows_core<A, S1, S2>(x, ar, t, j, k1, lr);
    }
    const uint64_t *cp = a.c + m * a.c_stride + (size_t)j * G::N + rowoff;
    const uint64_t *bp = (m & 1u) ? a.base1 : a.base0;
    if (bp) bp += (size_t)(m >> 1) * a.base_stride + (size_t)j * G::N + rowoff;
    const ulonglong2 f = a.f[j];
    uint64_t *op = a.out + lo;
    // The c and base values of a group of EG elements are requested before the
    // group's first store: the output may alias the base, so loads interleaved
    // with the stores would each be waited for in turn (one load in flight per
    // wave).  Each thread reads and writes only its own positions, so this is
    // safe; groups of 8 keep the registers those values take in bounds.
    constexpr int EG = SB::E < 8 ? SB::E : 8;
    const ulonglong2 f1 = a.f1 ? a.f1[j] : ulonglong2{0, 0};
#pragma unroll
    for (int e0 = 0; e0 < SB::E; e0 += EG) {
        uint64_t cv[EG], bv[EG];
#pragma unroll
        for (int i = 0; i < EG; i++) cv[i] = ld_stream(&cp[SB::T * (e0 + i)]);
#pragma unroll
        for (int i = 0; i < EG; i++) bv[i] = bp ? ld_stream(&bp[SB::T * (e0 + i)]) : 0;
#pragma unroll
        for (int i = 0; i < EG; i++) {
            const int e = e0 + i;
            uint64_t v;
            if (a.f1) {
                if constexpr (A::kF64) {
                    ar.reduce(x[e]);
                    double d = ar.load(cv[i]);
                    ar.mul(d, f1);
                    d += ar.load(bv[i]) - x[e];
                    ar.mul(d, f);
                    v = ar.store(d);
                } else {
                    const uint64_t cf = shoup(cv[i], f1.x, f1.y, ar.q);
                    const uint64_t d = sub_mod(add_mod(cf, bv[i], ar.q), ar.store(x[e]), ar.q);
                    v = shoup(d, f.x, f.y, ar.q);
                }
            } else if constexpr (A::kF64) {
                ar.reduce(x[e]);
                double d = ar.load(cv[i]) - x[e];
                ar.mul(d, f);
                v = ar.store(d);
                if (bp) v = add_mod(v, bv[i], (uint64_t)ar.q);
            } else {
                const uint64_t d = sub_mod(cv[i], ar.store(x[e]), ar.q);
                v = shoup(d, f.x, f.y, ar.q);
                if (bp) v = add_mod(v, bv[i], ar.q);
            }
            st_stream(&op[SB::T * e], v);
        }
    }
}

template <int S1, int S2>
__global__ void __launch_bounds__((FGeo<S1, S2>::THREADS))
k_epi_rows(EpiRows a, NttTables t) {
    using G = Geo<S1, S2>;
    using FG = FGeo<S1, S2>;
    __shared__ double lds[FG::LDS];
    __shared__ ulonglong2 twl[S2 * FG::ROWS + (1 << (S2 - 1))];
    const uint32_t rr = threadIdx.x / Sub<S2>::T;
    const uint32_t total = a.M * a.J * FG::TILES;
    for (uint32_t p = blockIdx.x; p < total; p += gridDim.x) {
        const uint32_t w = a.sched ? ld_const(a.sched + p) : p;
        const uint32_t tile = w % FG::TILES, mj = w / FG::TILES;
        const uint32_t m = mj % a.M, j = mj / a.M;
        const uint64_t q = t.mod[j];
        const uint32_t k1 = tile * FG::ROWS + rr;
        if (q < kF64PrimeBound)
            epi_item<ArithF64, S1, S2>(a, t, ArithF64(q), m, j, k1, lds + rr * G::ROW_PITCH, twl);
        else
            epi_item<ArithInt, S1, S2>(a, t, ArithInt(q), m, j, k1,
                                       reinterpret_cast<uint64_t *>(lds) + rr * G::ROW_PITCH, twl);
        __syncthreads();
    }
}

// ------------------------------------------------------------ rescale's last limb
// Fused ModDown + rescale: over M groups of [1 + alpha][N] coefficient-form
// limbs x (x_0 = INTT(base + cx [P^-1]) of the last limb, x_(1+i) = the scaled
// INTT of P limb i), x_0 := (x_0 - sum_i x_(1+i) g_i) mod q with
// g_i = [p_i^-1]_q: the canonical coefficients of the ModDown output's last
// limb.  128-bit products, one Barrett reduction (alpha < 64 keeps the sum
// below 2^128 for residues below 2^61).
__global__ void k_mdr_last(uint64_t *x, const uint64_t *g, const uint64_t *mod, const ulonglong2 *ratio,
                           uint32_t row, uint32_t alpha, uint32_t N, uint32_t M) {
    const uint64_t q = mod[row];
    const ulonglong2 rt = ratio[row];
    const uint32_t total = M * N;
    for (uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += gridDim.x * blockDim.x) {
        const uint32_t m = idx / N, k = idx % N;
        uint64_t *base = x + (size_t)m * (alpha + 1) * N + k;
        // the limbs' values are requested before the first product, 8 at a time
        // (a rolled loop waited for each value before requesting the next)
        const uint64_t x0 = base[0];
        U128 acc{0, 0};
        for (uint32_t i0 = 0; i0 < alpha; i0 += 8) {
            uint64_t v[8];
#pragma unroll
            for (uint32_t u = 0; u < 8; u++)
                if (i0 + u < alpha) v[u] = base[(size_t)(i0 + u + 1) * N];
#pragma unroll
            for (uint32_t u = 0; u < 8; u++)
                if (i0 + u < alpha) mac(acc, v[u], ld_const(g + i0 + u));
        }
        base[0] = sub_mod(x0, barrett128(acc, q, rt.x, rt.y), q);
    }
}

// ------------------------------------------------------------ tensor + INTT rows
// The HMult's tensor product with the first pass of the key switch's INTT(d2)
// fused in.  One workgroup per (member, limb, tile of R rows); a tile's R N2
// residues are contiguous in the limb, so the tensor reads and writes them with
// 16-byte accesses, thread t taking pairs 2t + 2 NT p.  d2 is still written in
// NTT form (the inner product reads its own-digit limbs from it) and goes
// through LDS into the inverse rows pass, whose output the inverse columns pass
// reads: d2 is not read back from HBM and the rows pass needs no launch of its
// own (the ModUp's INTT over Ql limbs is a fraction of a round of tiles).
struct TensorRows {
    const uint64_t *a, *b;
    uint64_t *d0, *d1, *d2, *mid;
    const ulonglong2 *ratio;
    uint32_t Ql, count;
    uint64_t in_stride, d_stride, d2_stride, mid_stride;
    const ulonglong2 *itw;  // set per workgroup: the tile's prime's inverse table
};

template <class A, int S1, int S2, int R, int MT>
__device__ __forceinline__ void tensor_rows_tile(const TensorRows &a, RowStage<S1, S2, R> &stage,
                                                 ulonglong2 *twl, const TileRef &r, uint64_t q,
                                                 typename A::T *lds) {
    using G = Geo<S1, S2>;
    using RS = RowStage<S1, S2, R>;
    // the tensor phase runs on all MT R T threads, the rows pass on the first R T
    constexpr uint32_t NR = R * Sub<S2>::T, NT = MT * NR;
    constexpr int P = Sub<S2>::E / 2 / MT, H = P / 2;
    static_assert(2 * NT * P == R * G::N2 && 2 * H == P, "a tile is NT threads x 2P residues");
    const A ar(q);
    ulonglong2 rt{0, 0};
    if constexpr (!A::kF64) rt = ld_const(a.ratio + r.l);
    // wave-uniform tile bases and a 32-bit per-thread index: the accesses
    // address scalar base + vector offset
    const size_t base = (size_t)r.l * G::N + (size_t)r.tile * R * G::N2;
    const uint64_t LN = (uint64_t)a.Ql * G::N;
    const uint64_t *pa0 = a.a + r.m * a.in_stride + base, *pb0 = a.b + r.m * a.in_stride + base;
    const uint64_t *pa1 = pa0 + LN, *pb1 = pb0 + LN;
    uint64_t *d0 = a.d0 + r.m * a.d_stride + base, *d1 = a.d1 + r.m * a.d_stride + base;
    uint64_t *d2 = a.d2 + r.m * a.d2_stride + base;
    // a window of W pairs in flight: pair k's products are stored as they are
    // formed and pair k + W is requested in their place (all 4P inputs at once
    // would need 8P VGPRs of loads alone); tile element i = 2 t + 2 NT p + h is
    // element i mod N2 of tile row i / N2
    constexpr int W = H;
    u64x2 a0[P], a1[P], b0[P], b1[P];
    const auto request = [&](int p) {
        const uint32_t j = 2 * threadIdx.x + 2 * NT * p;
        a0[p] = ld_stream2(pa0 + j);
        a1[p] = ld_stream2(pa1 + j);
        b0[p] = ld_stream2(pb0 + j);
        b1[p] = ld_stream2(pb1 + j);
    };
#pragma unroll
    for (int p = 0; p < W; p++) request(p);
    // visible to the rounds after the barrier that follows the LDS fill
    stage.st.store(twl);
#pragma unroll
    for (int p = 0; p < P; p++) {
        uint64_t r0[2], r1[2], r2[2];
#pragma unroll
        for (int h = 0; h < 2; h++) {
            if constexpr (A::kF64)
                tensor_elem(ar, a0[p][h], a1[p][h], b0[p][h], b1[p][h], r0[h], r1[h], r2[h]);
            else
                tensor_elem(q, rt, a0[p][h], a1[p][h], b0[p][h], b1[p][h], r0[h], r1[h], r2[h]);
        }
        const uint32_t j = 2 * threadIdx.x + 2 * NT * p;
        st_stream2(d0 + j, r0[0], r0[1]);
        st_stream2(d1 + j, r1[0], r1[1]);
        st_stream2(d2 + j, r2[0], r2[1]);
        if (p + W < P) request(p + W);
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const uint32_t i = j + h;
            lds[(i / G::N2) * G::ROW_PITCH + rpad(i % G::N2)] = ar.load(r2[h]);
        }
    }
    __syncthreads();
    const TileTw w = RS::view(twl, a.itw, threadIdx.x / Sub<S2>::T);
    inv_rows_lds<A, S1, S2, R, true, R>(w, r, q, lds, a.mid + r.m * a.mid_stride + (size_t)r.l * G::N,
                                        threadIdx.x < NR);
}

template <int S1, int S2, int R, int MT>
__global__ void __launch_bounds__(MT * R * Sub<S2>::T) __attribute__((amdgpu_waves_per_eu(4, 8)))
k_tensor_rows(TensorRows a, NttTables t) {
    using G = Geo<S1, S2>;
    using RS = RowStage<S1, S2, R>;
    constexpr uint32_t TILES = G::N1 / R;
    __shared__ double lds[R * G::ROW_PITCH];
    __shared__ ulonglong2 twl[RS::N];
    const TileRef r{blockIdx.y, blockIdx.x / TILES, blockIdx.x % TILES};
    const uint64_t q = ld_const(t.mod + r.l);
    a.itw = t.itw + (size_t)r.l * G::N;
    // the tile's twiddle factors are requested before its residues
    RS stage;
    stage.load(t, r.l, r.tile, false);
    if (q < kF64PrimeBound)
        tensor_rows_tile<ArithF64, S1, S2, R, MT>(a, stage, twl, r, q, lds);
    else
        tensor_rows_tile<ArithInt, S1, S2, R, MT>(a, stage, twl, r, q, reinterpret_cast<uint64_t *>(lds));
}

// ------------------------------------------------------------ launchers
NttTables tables_of(const Ctx &c) {
    return NttTables{c.mod, c.tw, c.itw, c.ninv, c.small_fw, c.small_inv, c.rb_fw, c.rb_inv};
}

uint32_t fgrid(const Ctx &c, uint32_t items, uint32_t wpc) {
    const uint32_t cap = (uint32_t)c.n_cu * wpc;
    return items < cap ? items : cap;
}

template <int S1, int S2>
void launch_bconv(const Ctx &c, const BconvCols &a0, hipStream_t s) {
    using G = Geo<S1, S2>;
    BconvCols a = a0;
    // the Montgomery-accumulated sums need sum_i t_i < 2^64; every input is
    // below the context's largest prime
    if (c.max_modulus <= ~0ull / std::max(a.n_in, a.n_in_last)) a.mont = c.mont;
    const uint32_t total = grouped_total(a.batch * a.groups * G::COL_TILES, a.J);
    const uint32_t grid = fgrid(c, total, 4);
    if (a.sched && (grid != a.sched_grid || total != a.sched_total)) a.sched = nullptr;
    hipLaunchKernelGGL((k_bconv_cols<S1, S2>), dim3(grid), dim3(G::COL_THREADS), 0, s, a, tables_of(c));
    PFA_HIP(hipGetLastError());
}

// Rows per tile: 8 for rows of 256 (N = 2^15, 2^16: 8 workgroups of 128
// threads fill a CU), the inverse rows pass's own height otherwise.
// The tensor phase of k_tensor_rows runs on twice the rows pass's threads
// (8 residues each instead of 16; the second half waits out the rows pass):
// its 1.5-2.2 waves per SIMD were too few to hide the loads (110 VGPRs,
// config-3 HMult 0.2753/0.2763/0.2759 -> 0.2733/0.2731/0.2734 ms, L = 35
// 0.7943/0.7940/0.7927 -> 0.7904/0.7896/0.7913 ms, interleaved on one box).
// The same split made the batch-1 rotation's Galois kernel slower (apply_galois
// 221.5/225.0/227.7 -> 225.3/231.2/233.0 us), so k_galois_rows keeps one.
constexpr int kTensorRowsMT = 2;
constexpr int kGaloisRowsMT = 1;

template <int S1, int S2>
void launch_tensor_rows(const Ctx &c, const TensorRows &a, hipStream_t s) {
    using G = Geo<S1, S2>;
    if constexpr (S2 > 8) {
        fail(PFA_ERR_INVALID_ARGUMENT, "fused tensor rows pass: N above 2^16");
    } else {
        constexpr int R = S2 == 8 && G::ROWS == 16 ? 8 : G::ROWS;
        constexpr int MT = kTensorRowsMT;
        hipLaunchKernelGGL((k_tensor_rows<S1, S2, R, MT>), dim3(a.Ql * (G::N1 / R), a.count),
                           dim3(MT * R * Sub<S2>::T), 0, s, a, tables_of(c));
        PFA_HIP(hipGetLastError());
    }
}

// largest number of split items one launch may have (arrival counters per workspace)
constexpr uint32_t kWsMaxSplit = 4096;

template <int S1, int S2>
void launch_inner(const Ctx &c, InnerRows a, hipStream_t s) {
    using G = Geo<S1, S2>;
    using W = WsGeo<S1, S2>;
    static const int occ = [] {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, (const void *)k_inner_ws<S1, S2>, W::THREADS, 0) !=
            hipSuccess)
            n = 1;
        return n > 0 ? n : 1;
    }();
    const uint32_t items = a.batch * a.QlP * W::TILES;
    const uint32_t P = c.ws_slots ? c.ws_slots : (uint32_t)c.n_cu * (uint32_t)occ;  // resident workgroups
    uint32_t grid = items;
    a.full = items;
    a.rem = 0;
    a.kch = 1;
    Scratch sc(c, s);
    if (items > P) {
        grid = P;
        const uint32_t rem = items % P;
        const uint32_t per_x = (rem + kXcds - 1) / kXcds;  // split items per XCD class
        // a split item's chunks run on workgroups congruent mod 8, which meet
        // in one XCD's L2 only where workgroups are dealt to the XCDs
        // round-robin (probed at context creation); elsewhere items run whole
        const uint32_t kch = rem && P % kXcds == 0 && c.xcd_rr ? std::min<uint32_t>(a.beta, (P / kXcds) / per_x) : 0;
        if (kch >= 2 && rem <= kWsMaxSplit) {
            Arena &ar = arena_for(c, s);
            if (!ar.ws_counter) {
                PFA_HIP(hipMalloc((void **)&ar.ws_counter, kWsMaxSplit * sizeof(uint32_t)));
                PFA_HIP(hipMemsetAsync(ar.ws_counter, 0, kWsMaxSplit * sizeof(uint32_t), s));
            }
            a.full = items - rem;
            a.rem = rem;
            a.kch = kch;
            a.partial = sc.alloc((size_t)rem * kch * 2 * W::ROWS * G::N2);
            a.counter = ar.ws_counter;
            a.host_err = c.err_host_dev;
        }
    }
    hipLaunchKernelGGL((k_inner_ws<S1, S2>), dim3(grid), dim3(W::THREADS), 0, s, a, tables_of(c));
    PFA_HIP(hipGetLastError());
}

template <int S1, int S2>
void launch_epi(const Ctx &c, const EpiRows &a0, hipStream_t s) {
    using FG = FGeo<S1, S2>;
    EpiRows a = a0;
    const uint32_t total = a.M * a.J * FG::TILES, grid = fgrid(c, total, 8);
    if (a.allow_sched) {
        const Sched sch = epi_schedule(c, a.J, a.M, FG::TILES, grid);
        if (sch.table && sch.grid == grid && sch.total == total) {
            a.sched = sch.table;
            a.sched_grid = sch.grid;
            a.sched_total = sch.total;
        }
    }
    hipLaunchKernelGGL((k_epi_rows<S1, S2>), dim3(grid), dim3(FG::THREADS), 0, s, a, tables_of(c));
    PFA_HIP(hipGetLastError());
}

#define PFA_FUSED_DISPATCH(FN, ARG)                                          \
    switch (c.logN) {                                                        \
    case 10: FN<5, 5>(c, ARG, s); break;                                     \
    case 11: FN<5, 6>(c, ARG, s); break;                                     \
    case 12: FN<6, 6>(c, ARG, s); break;                                     \
    case 13: FN<6, 7>(c, ARG, s); break;                                     \
    case 14: FN<7, 7>(c, ARG, s); break;                                     \
    case 15: FN<7, 8>(c, ARG, s); break;                                     \
    case 16: FN<8, 8>(c, ARG, s); break;                                     \
    case 17: FN<8, 9>(c, ARG, s); break;                                     \
    default: fail(PFA_ERR_INVALID_ARGUMENT, "unsupported poly_modulus_degree"); \
    }

}  // namespace

// c2 [Ql][N] (NTT form) -> cx [2][QlP][N]: ModUp and the key-switch inner
// product against key [dnum][2][QP][N].
// The ModUp of batch members c2 (+ i c2_stride) up to the forward NTT's
// columns pass: the scaled INTT, then the base conversion fused with the
// columns pass into inter [batch][beta][QlP][N] (each digit's own limbs not
// written).  With c2_mid the INTT runs its columns pass only, on c2_mid.
static void modup_cols(const Ctx &c, uint32_t chain, const uint64_t *c2, uint64_t c2_stride, const uint64_t *c2_mid,
                       uint64_t *inter, uint32_t batch, hipStream_t s) {
    const Level &lv = c.level(chain);
    const uint32_t Ql = lv.Ql, alpha = c.P, QlP = Ql + alpha;
    const uint64_t LN = (uint64_t)Ql * c.N, IN = (uint64_t)lv.beta * QlP * c.N;
    Scratch sc(c, s);
    uint64_t *tin = sc.alloc((size_t)batch * LN);
    if (c2_mid) {
        NttLaunch inv{c2_mid, tin, LN, LN, batch, Ql};
        inv.scale = lv.modup_scale;
        ntt_inverse_cols(c, inv, s);
    } else {
        NttLaunch inv{c2, tin, c2_stride, LN, batch, Ql};
        inv.scale = lv.modup_scale;
        ntt_inverse(c, inv, s);
    }
    BconvCols b{};
    b.in = tin;
    b.out = inter;
    b.bc = lv.modup_bc;
    b.in_gstride = (uint64_t)alpha * c.N;
    b.out_gstride = (uint64_t)QlP * c.N;
    b.groups = lv.beta;
    b.J = QlP;
    b.n_in = alpha;
    b.n_in_last = Ql - (lv.beta - 1) * alpha;
    b.in_row0 = 0;
    b.in_row_step = alpha;
    b.split = Ql;
    b.split_base = c.Q;
    b.skip = 1;
    b.bc_gstride = 2 * alpha * QlP;
    b.bc_istride = QlP;
    b.unit = alpha == 1;
    b.batch = batch;
    b.in_bstride = LN;
    b.out_bstride = IN;
    const Sched sch = modup_schedule(c, chain, batch);
    b.sched = sch.table;
    b.sched_grid = sch.grid;
    b.sched_total = sch.total;
    PFA_FUSED_DISPATCH(launch_bconv, b);
}

void fused_modup_ntt(const Ctx &c, uint32_t chain, const uint64_t *c2, uint64_t *out, hipStream_t s) {
    const Level &lv = c.level(chain);
    const uint32_t QlP = lv.Ql + c.P;
    modup_cols(c, chain, c2, 0, nullptr, out, 1, s);
    NttLaunch fw{out, out, (uint64_t)QlP * c.N, (uint64_t)QlP * c.N, lv.beta, QlP};
    fw.start = 0;
    fw.split = lv.Ql;
    fw.split_base = c.Q;
    fw.ex_lo = 0;
    fw.ex_step = c.P;
    fw.ex_len = c.P;
    fw.ex_cap = lv.Ql;
    ntt_forward_rows(c, fw, s);
}

void fused_modup_inner(const Ctx &c, uint32_t chain, const uint64_t *c2, const uint64_t *key, uint64_t *cx,
                       hipStream_t s, uint32_t batch, uint64_t c2_stride, uint64_t cx_stride, const KsFold *fold,
                       const uint64_t *const *key_table, const uint64_t *c2_mid) {
    const Level &lv = c.level(chain);
    const uint32_t Ql = lv.Ql, alpha = c.P, QlP = Ql + alpha;
    const uint64_t IN = (uint64_t)lv.beta * QlP * c.N;
    Scratch sc(c, s);
    uint64_t *inter = sc.alloc((size_t)batch * IN);
    modup_cols(c, chain, c2, c2_stride, c2_mid, inter, batch, s);
    InnerRows r{inter, c2, key, cx, c.mont, Ql, QlP, alpha, lv.beta, c.Q, c.QP};
    r.batch = batch;
    r.inter_bstride = IN;
    r.c2_bstride = c2_stride;
    r.cx_bstride = cx_stride ? cx_stride : (uint64_t)2 * QlP * c.N;
    r.key_table = key_table;
    // one key for all members: interleave them so they share its rows in L2
    r.member_fast = batch > 1 && !key_table ? 1u : 0u;
    if (batch == 1) r.order = lv.ws_order;
    if (fold) {
        require(fold->base0 && fold->base1 && Ql >= 2 && (batch == 1 || fold->stride), "bad ModDown + rescale fold");
        r.fold_r = Ql - 1;
        r.fold_base0 = fold->base0;
        r.fold_base1 = fold->base1;
        r.fold_bstride = fold->stride;
        r.fold_f = c.pinv + (Ql - 1);
    }
    PFA_FUSED_DISPATCH(launch_inner, r);
}

void fused_tensor_rows(const Ctx &c, uint32_t chain, const uint64_t *a, const uint64_t *b, uint64_t *d0,
                       uint64_t *d1, uint64_t *d2, uint64_t *mid, hipStream_t s, uint32_t count,
                       uint64_t in_stride, uint64_t d_stride, uint64_t d2_stride) {
    const uint32_t Ql = c.level(chain).Ql;
    require(c.logN <= 16, "fused tensor rows pass: N above 2^16");
    require(count >= 1 && (count == 1 || (in_stride && d_stride && d2_stride)), "bad tensor batch");
    require(((uintptr_t)a | (uintptr_t)b | (uintptr_t)d0 | (uintptr_t)d1 | (uintptr_t)d2 | (uintptr_t)mid) % 16 == 0 &&
                (in_stride | d_stride | d2_stride) % 2 == 0,
            "tensor operands must be 16-byte aligned");
    const TensorRows t{a, b, d0, d1, d2, mid, c.ratio, Ql, count, in_stride, d_stride, d2_stride, (uint64_t)Ql * c.N,
                       nullptr};
    PFA_FUSED_DISPATCH(launch_tensor_rows, t);
}

// ------------------------------------------------------------ rotation input
// Both polys of B ciphertexts through the Galois permutation of NTT slots
// (apply_galois_ntt_permutation, src/galois.cu:11-18), with the first pass of
// the key switch's INTT fused in for poly 1 (the c2 that apply_galois_with_ksk
// key-switches, src/evaluate.cu:1607-1656):
//   dst[i][k][l][n] = src[i][k][l][pi_i(n)]  (+ add0[l][n] for k = 0, B = 1)
//   mid[i][l]       = inverse rows pass of dst[i][1][l]
// A tile is R rows of one limb of one poly: its residues are gathered (the
// permutation stays within the limb), stored, and for poly 1 also placed in
// LDS, where the inverse rows pass takes them as k_tensor_rows does.
struct GaloisRows {
    const uint64_t *src;
    uint64_t src_stride;
    uint64_t *dst;          // [B][2][Ql][N]
    const uint64_t *add0;   // [Ql][N] or null
    uint64_t *mid;          // [B][Ql][N]
    const uint32_t *elts;   // [B] device table, or null: every member uses elt
    uint32_t elt, Ql, logN, B;
};

template <int S1, int S2, int R, int MT>
__global__ void __launch_bounds__(MT * R * Sub<S2>::T) __attribute__((amdgpu_waves_per_eu(3, 8)))
k_galois_rows(GaloisRows a, NttTables t) {
    using G = Geo<S1, S2>;
    using RS = RowStage<S1, S2, R>;
    // the gathers run on all MT R T threads, the rows pass on the first R T
    constexpr uint32_t TILES = G::N1 / R, NR = R * Sub<S2>::T, NT = MT * NR, E = Sub<S2>::E / MT;
    static_assert(NT * E == R * G::N2, "a tile is NT threads x E residues");
    __shared__ double lds[R * G::ROW_PITCH];
    __shared__ ulonglong2 twl[RS::N];
    const uint32_t k = blockIdx.y & 1u, i = blockIdx.y >> 1;
    const TileRef r{i, blockIdx.x / TILES, blockIdx.x % TILES};
    const uint64_t q = ld_const(t.mod + r.l);
    const uint32_t e = a.elts ? uniform_u32(a.elts[i]) : a.elt;
    const size_t row = ((size_t)k * a.Ql + r.l) * G::N;
    const uint32_t tb = r.tile * R * G::N2;  // first element of the tile within the limb
    const uint64_t *src = a.src + i * a.src_stride + row;
    uint64_t *dst = a.dst + (size_t)i * 2 * a.Ql * G::N + row + tb;
    RS stage;
    if (k) stage.load(t, r.l, r.tile, false);  // requested before the residues
    uint64_t v[E];
#pragma unroll
    for (uint32_t p = 0; p < E; p++) v[p] = src[galois_perm(e, tb + threadIdx.x + NT * p, a.logN)];
    if (!k) {
        if (a.add0) {
            const uint64_t *ad = a.add0 + (size_t)r.l * G::N + tb;
#pragma unroll
            for (uint32_t p = 0; p < E; p++) v[p] = add_mod(v[p], ad[threadIdx.x + NT * p], q);
        }
#pragma unroll
        for (uint32_t p = 0; p < E; p++) st_stream(dst + threadIdx.x + NT * p, v[p]);
        return;
    }
    // the staged twiddles were requested first: this waits for them only
    stage.st.store(twl);
    uint64_t *mid = a.mid + ((size_t)i * a.Ql + r.l) * G::N;
    const TileTw w = RS::view(twl, t.itw + (size_t)r.l * G::N, threadIdx.x / Sub<S2>::T);
    if (q < kF64PrimeBound) {
        const ArithF64 ar(q);
#pragma unroll
        for (uint32_t p = 0; p < E; p++) {
            const uint32_t j = threadIdx.x + NT * p;
            st_stream(dst + j, v[p]);
            lds[(j / G::N2) * G::ROW_PITCH + rpad(j % G::N2)] = ar.load(v[p]);
        }
        __syncthreads();
        inv_rows_lds<ArithF64, S1, S2, R, true, R>(w, r, q, lds, mid, threadIdx.x < NR);
    } else {
        const ArithInt ar(q);
        uint64_t *li = reinterpret_cast<uint64_t *>(lds);
#pragma unroll
        for (uint32_t p = 0; p < E; p++) {
            const uint32_t j = threadIdx.x + NT * p;
            st_stream(dst + j, v[p]);
            li[(j / G::N2) * G::ROW_PITCH + rpad(j % G::N2)] = ar.load(v[p]);
        }
        __syncthreads();
        inv_rows_lds<ArithInt, S1, S2, R, true, R>(w, r, q, li, mid, threadIdx.x < NR);
    }
}

template <int S1, int S2>
void launch_galois_rows(const Ctx &c, const GaloisRows &a, hipStream_t s) {
    using G = Geo<S1, S2>;
    if constexpr (S2 > 8) {
        fail(PFA_ERR_INVALID_ARGUMENT, "fused Galois rows pass: N above 2^16");
    } else {
        constexpr int R = S2 == 8 && G::ROWS == 16 ? 8 : G::ROWS;
        constexpr int MT = kGaloisRowsMT;
        hipLaunchKernelGGL((k_galois_rows<S1, S2, R, MT>), dim3(a.Ql * (G::N1 / R), 2 * a.B),
                           dim3(MT * R * Sub<S2>::T), 0, s, a, tables_of(c));
        PFA_HIP(hipGetLastError());
    }
}

void galois_rows(const Ctx &c, uint32_t chain, const uint64_t *src, uint64_t src_stride, uint32_t B, uint32_t elt,
                 const uint32_t *elts, const uint64_t *add0, uint64_t *dst, uint64_t *mid, hipStream_t s) {
    const uint32_t Ql = c.size_Ql(chain);
    require(c.logN <= 16, "fused Galois rows pass: N above 2^16");
    require(B >= 1 && B <= 32767, "bad rotation batch");
    const GaloisRows g{src, src_stride, dst, add0, mid, elts, elt, Ql, c.logN, B};
    PFA_FUSED_DISPATCH(launch_galois_rows, g);
}

// The rescale of base + ModDown(cx) without forming the ModDown output.  With
// q_l the last prime, v_i the scaled INTT of P limb i and
// t = INTT(base + cx [P^-1])_(l) - sum_i v_i [p_i^-1]_(q_l) mod q_l (the
// ModDown output's last limb in coefficient form), for j < l:
//   out_j = (cx_j [P^-1] + base_j - NTT(sum_i v_i [p_i^-1]_(q_j) + t)) [q_l^-1]
// which is ModDown's (cx - NTT(delta)) P^-1 + base followed by the rescale's
// (c - NTT(t mod q_j)) q_l^-1 with the two NTTs merged by linearity.
void fused_moddown_rescale(const Ctx &c, uint32_t chain, const uint64_t *cx, const uint64_t *base0,
                           const uint64_t *base1, uint64_t *out, hipStream_t s, uint32_t count,
                           uint64_t base_stride) {
    const Level &lv = c.level(chain);
    const uint32_t Ql = lv.Ql, alpha = c.P, QlP = Ql + alpha, J = Ql - 1, M = 2 * count;
    require(Ql >= 2, "cannot rescale at the last level");
    require(count >= 1 && (count == 1 || base_stride), "bad ModDown + rescale batch");
    Scratch sc(c, s);
    uint64_t *x = sc.alloc((size_t)M * (alpha + 1) * c.N);
    uint64_t *inter = sc.alloc((size_t)M * J * c.N);
    NttLaunch inv{cx + (size_t)(Ql - 1) * c.N, x, (uint64_t)QlP * c.N, (uint64_t)(alpha + 1) * c.N, M, alpha + 1};
    inv.start = Ql - 1;
    inv.split = 1;
    inv.split_base = c.Q;
    inv.scale = lv.mdr_scale;
    ntt_inverse(c, inv, s);
    hipLaunchKernelGGL(k_mdr_last, dim3((M * c.N + 255) / 256), dim3(256), 0, s, x, lv.mdr_glast, c.mod, c.ratio,
                       Ql - 1, alpha, c.N, M);
    PFA_HIP(hipGetLastError());
    BconvCols b{};
    b.in = x;
    b.out = inter;
    b.bc = c.mdr_bc;
    b.in_gstride = (uint64_t)(alpha + 1) * c.N;
    b.out_gstride = (uint64_t)J * c.N;
    b.groups = M;
    b.J = J;
    b.n_in = alpha + 1;
    b.n_in_last = alpha + 1;
    b.in_row0 = c.Q;
    b.in_row_step = 0;
    b.first_row = Ql - 1;
    b.split = 0xffffffffu;
    b.split_base = 0;
    b.skip = 0;
    b.bc_gstride = 0;
    b.bc_istride = c.Q;
    PFA_FUSED_DISPATCH(launch_bconv, b);
    EpiRows e{inter, cx, base0, base1, out, lv.rescale_inv_p, (uint64_t)QlP * c.N, M, J};
    e.base_stride = base_stride;
    e.f1 = c.pinv_p;
    PFA_FUSED_DISPATCH(launch_epi, e);
}

// cx [M][QlP][N] -> out [M][Ql][N] = base + ModDown(cx): poly 2i + k adds
// base_k + i base_stride (base_k may alias out's polys or be null)
void fused_moddown(const Ctx &c, uint32_t chain, const uint64_t *cx, uint32_t M, uint64_t *out,
                   const uint64_t *base0, const uint64_t *base1, hipStream_t s, uint64_t base_stride) {
    const uint32_t Ql = c.size_Ql(chain), alpha = c.P, QlP = Ql + alpha;
    Scratch sc(c, s);
    uint64_t *xP = sc.alloc((size_t)M * alpha * c.N);
    uint64_t *inter = sc.alloc((size_t)M * Ql * c.N);
    NttLaunch inv{cx + (size_t)Ql * c.N, xP, (uint64_t)QlP * c.N, (uint64_t)alpha * c.N, M, alpha};
    inv.start = c.Q;
    inv.scale = c.moddown_scale;
    ntt_inverse(c, inv, s);
    BconvCols b{};
    b.in = xP;
    b.out = inter;
    b.bc = c.moddown_bc;
    b.in_gstride = (uint64_t)alpha * c.N;
    b.out_gstride = (uint64_t)Ql * c.N;
    b.groups = M;
    b.J = Ql;
    b.n_in = alpha;
    b.n_in_last = alpha;
    b.in_row0 = c.Q;
    b.in_row_step = 0;
    b.split = 0xffffffffu;
    b.split_base = 0;
    b.skip = 0;
    b.bc_gstride = 0;
    b.bc_istride = c.Q;
    PFA_FUSED_DISPATCH(launch_bconv, b);
    EpiRows e{inter, cx, base0, base1, out, c.pinv_p, (uint64_t)QlP * c.N, M, Ql};
    e.base_stride = base_stride;
    PFA_FUSED_DISPATCH(launch_epi, e);
}

// in [size][L][N] -> out [size][L-1][N]: floor division by the last prime
void fused_rescale(const Ctx &c, uint32_t chain, const uint64_t *in, uint32_t size, uint64_t *out, hipStream_t s) {
    const uint32_t L = c.level(chain).Ql;
    Scratch sc(c, s);
    uint64_t *last = sc.alloc((size_t)size * c.N);
    uint64_t *inter = sc.alloc((size_t)size * (L - 1) * c.N);
    fused_rescale_with(c, chain, in, size, out, last, inter, s, true);
}

void fused_rescale_with(const Ctx &c, uint32_t chain, const uint64_t *in, uint32_t size, uint64_t *out,
                        uint64_t *last, uint64_t *inter, hipStream_t s, bool allow_flow) {
    const Level &lv = c.level(chain);
    const uint32_t L = lv.Ql;
    NttLaunch inv{in + (size_t)(L - 1) * c.N, last, (uint64_t)L * c.N, (uint64_t)c.N, size, 1};
    inv.start = L - 1;
    ntt_inverse(c, inv, s, allow_flow);
    BconvCols b{};
    b.in = last;
    b.out = inter;
    b.bc = c.unit_bc;
    b.unit = 1;
    b.in_gstride = c.N;
    b.out_gstride = (uint64_t)(L - 1) * c.N;
    b.groups = size;
    b.J = L - 1;
    b.n_in = 1;
    b.n_in_last = 1;
    b.in_row0 = L - 1;
    b.in_row_step = 0;
    b.split = 0xffffffffu;
    b.split_base = 0;
    b.skip = 0;
    b.bc_gstride = 0;
    b.bc_istride = 0;
    PFA_FUSED_DISPATCH(launch_bconv, b);
    EpiRows e{inter, in, nullptr, nullptr, out, lv.rescale_inv_p, (uint64_t)L * c.N, size, L - 1};
    e.allow_sched = allow_flow;
    PFA_FUSED_DISPATCH(launch_epi, e);
}

}  // namespace pfa
