// NTT launchers and the raw-limb NTT entry points of the C ABI.
#include <algorithm>
#include <cstdlib>
#include <vector>

#include "internal.h"
#include "ntt_kernels.h"

namespace pfa {

namespace {

NttBatch make_batch(const Ctx &c, const NttLaunch &a) {
    NttBatch b;
    b.src = a.src;
    b.dst = a.dst;
    b.sstride = a.sstride ? a.sstride : (uint64_t)a.L * c.N;
    b.dstride = a.dstride ? a.dstride : (uint64_t)a.L * c.N;
    b.M = a.M;
    b.L = a.L;
    b.map = LimbMap{a.start, a.split, a.split_base};
    b.ex_lo = a.ex_lo;
    b.ex_step = a.ex_step;
    b.ex_len = a.ex_len;
    b.ex_cap = a.ex_cap;
    b.scale = a.scale;
    return b;
}

NttTables tables(const Ctx &c) {
    return NttTables{c.mod, c.tw, c.itw, c.ninv, c.small_fw, c.small_inv, c.rb_fw, c.rb_inv};
}

// persistent grid: at most n_cu * wpc workgroups, each walking its tiles
// (wpc: ntt_wpc for the inverse passes, ntt_wpc_fwd for the forward ones)
uint32_t grid_for(const Ctx &c, uint32_t tiles, int wpc) {
    const uint32_t cap = (uint32_t)c.n_cu * (uint32_t)wpc;
    return tiles < cap ? tiles : cap;
}

// Rows per tile of the forward rows pass: 8 instead of 16 for rows of 256
// (N = 2^15 and 2^16; 8 workgroups of 128 threads and 20 KiB of LDS fill a
// CU, the other shapes keep their tiles).  The config-2 batch then has 2240
// tiles of 8 rows for 2048 resident workgroups (8 per CU) instead of 1120 of
// 16 rows for 1024: the tiles dealt beyond one per workgroup are a smaller
// share of a CU's work (measured on the 2 x 35-limb batch, five interleaved
// pairs: rows pass 20.4 -> 19.5 us).  The staged inverse rows pass (batches of
// 48 limbs or more) measured the same with either height and keeps 16; the
// prefetching one (the key switch's INTTs, 6 workgroups per CU) takes 8 rows:
// L = 35 HMult 0.800 / 0.801 -> 0.797 / 0.798 ms, config 3 unchanged.
template <int S1, int S2>
constexpr int half_rows() {
    using G = Geo<S1, S2>;
    return S2 == 8 && G::ROWS == 16 ? 8 : G::ROWS;
}

// the forward rows pass alone: b.src holds a columns pass's output
template <int S1, int S2>
void fwd_rows(const Ctx &c, const NttBatch &b, const NttTables &t, hipStream_t s) {
    using G = Geo<S1, S2>;
    const uint32_t ml = b.M * b.L;
    constexpr int RH = half_rows<S1, S2>();
    if (RH != G::ROWS)
        hipLaunchKernelGGL((ntt_fwd_rows<S1, S2, RH>), dim3(grid_for(c, ml * (G::N1 / RH), c.ntt_wpc_fwd * (G::ROWS / RH))),
                           dim3(RH * Sub<S2>::T), 0, s, b, t);
    else
        hipLaunchKernelGGL((ntt_fwd_rows<S1, S2>), dim3(grid_for(c, ml * G::ROW_TILES, c.ntt_wpc_fwd)), dim3(G::ROW_THREADS), 0, s, b,
                           t);
}

template <int S1, int S2>
void fwd(const Ctx &c, const NttBatch &b, const NttTables &t, hipStream_t s) {
    using G = Geo<S1, S2>;
    const uint32_t ml = b.M * b.L;
    hipLaunchKernelGGL((ntt_fwd_cols<S1, S2>), dim3(grid_for(c, ml * G::COL_TILES, c.ntt_wpc_fwd)), dim3(G::COL_THREADS), 0, s, b,
                       t);
    NttBatch b2 = b;
    b2.src = b.dst;
    b2.sstride = b.dstride;
    fwd_rows<S1, S2>(c, b2, t, s);
}

// batches of at least this many limbs take the inverse rows pass with staged twiddles
constexpr uint32_t kInvStagedLimbs = 48;

// the inverse columns pass alone: b.src holds the rows pass's output
template <int S1, int S2>
void inv_cols(const Ctx &c, const NttBatch &b, const NttTables &t, hipStream_t s) {
    using G = Geo<S1, S2>;
    hipLaunchKernelGGL((ntt_inv_cols<S1, S2>), dim3(grid_for(c, b.M * b.L * G::COL_TILES, c.ntt_wpc_fwd)),
                       dim3(G::COL_THREADS), 0, s, b, t);
}

template <int S1, int S2>
void inv(const Ctx &c, const NttBatch &b, const NttTables &t, hipStream_t s) {
    using G = Geo<S1, S2>;
    const uint32_t ml = b.M * b.L;
    if (ml >= kInvStagedLimbs)
        hipLaunchKernelGGL((ntt_inv_rows_staged<S1, S2>), dim3(grid_for(c, ml * G::ROW_TILES, 3)),
                           dim3(G::ROW_THREADS), 0, s, b, t);
    else if (half_rows<S1, S2>() != G::ROWS)
        hipLaunchKernelGGL((ntt_inv_rows<S1, S2, half_rows<S1, S2>()>),
                           dim3(grid_for(c, ml * (G::N1 / half_rows<S1, S2>()), c.ntt_wpc * (G::ROWS / half_rows<S1, S2>()))),
                           dim3(half_rows<S1, S2>() * Sub<S2>::T), 0, s, b, t);
    else
        hipLaunchKernelGGL((ntt_inv_rows<S1, S2>), dim3(grid_for(c, ml * G::ROW_TILES, c.ntt_wpc)),
                           dim3(G::ROW_THREADS), 0, s, b, t);
    NttBatch b2 = b;
    b2.src = b.dst;
    b2.sstride = b.dstride;
    inv_cols<S1, S2>(c, b2, t, s);
}

void check_launch(const Ctx &c, const NttLaunch &a) {
    require(a.src && a.dst, "null data pointer");
    require(a.M >= 1 && a.L >= 1, "empty batch");
    if (a.M > 1) {
        require(a.sstride == 0 || a.sstride >= (uint64_t)a.L * c.N, "poly stride smaller than one poly");
        require(a.dstride == 0 || a.dstride >= (uint64_t)a.L * c.N, "poly stride smaller than one poly");
    }
    require((uint64_t)a.M * a.L * (c.N / 16) < (1ULL << 31), "batch too large for one launch");
    // every limb must map to a table row inside the context
    const uint32_t last = a.L - 1;
    const uint32_t rlast = last < a.split ? a.start + last : a.split_base + (last - a.split);
    const uint32_t rfirst = 0 < a.split ? a.start : a.split_base;
    require(rfirst < c.QP && rlast < c.QP, "limb range exceeds the context's primes");
    if (a.split < a.L) require(a.start + a.split <= c.QP, "limb range exceeds the context's primes");
}

}  // namespace

// Single-launch transform (N = 2^16; see ntt_kernels.h).  Takes the next of
// the two control blocks of the calling thread's workspace for stream s.
template <bool FWD>
void flow(const Ctx &c, const NttBatch &b, const NttTables &t, hipStream_t s) {
    const uint32_t jobs = b.M * b.L;
    Arena &a = arena_for(c, s);
    if (!a.flow) {
        PFA_HIP(hipMalloc((void **)&a.flow, 2 * (size_t)kFlowBlockWords * sizeof(uint32_t)));
        PFA_HIP(hipMemsetAsync(a.flow, 0, 2 * (size_t)kFlowBlockWords * sizeof(uint32_t), s));
    }
    const uint32_t p = a.flow_parity;
    FlowCtl f;
    f.blk = a.flow + (size_t)p * kFlowBlockWords;
    f.other = a.flow + (size_t)(1 - p) * kFlowBlockWords;
    f.other_jobs = a.flow_dirty[1 - p];
    f.window = c.flow_window;
    f.wait_ticks = c.flow_wait_ticks;
    f.host_err = c.err_host_dev;
    const uint32_t grid = (uint32_t)c.n_cu * (uint32_t)c.flow_wpc / kXcds * kXcds;
    if (FWD) {
        if (c.flow_wpc >= 4)
            hipLaunchKernelGGL((ntt_fwd_flow<8, 8, 4>), dim3(grid), dim3(256), 0, s, b, t, f);
        else
            hipLaunchKernelGGL((ntt_fwd_flow<8, 8, 3>), dim3(grid), dim3(256), 0, s, b, t, f);
    } else {
        if (c.flow_wpc >= 4)
            hipLaunchKernelGGL((ntt_inv_flow<8, 8, 4>), dim3(grid), dim3(256), 0, s, b, t, f);
        else
            hipLaunchKernelGGL((ntt_inv_flow<8, 8, 3>), dim3(grid), dim3(256), 0, s, b, t, f);
    }
    PFA_HIP(hipGetLastError());
    a.flow_parity = 1 - p;
    a.flow_dirty[p] = jobs;
    a.flow_dirty[1 - p] = 0;
}

bool use_flow(const Ctx &c, const NttBatch &b) {
    const uint32_t jobs = b.M * b.L;
    return c.ntt_flow && c.logN == 16 && jobs >= c.flow_min_jobs && jobs <= kFlowMaxJobs;
}

#define PFA_NTT_DISPATCH(FN)                                                 \
    switch (c.logN) {                                                        \
    case 10: FN<5, 5>(c, b, t, s); break;                                       \
    case 11: FN<5, 6>(c, b, t, s); break;                                       \
    case 12: FN<6, 6>(c, b, t, s); break;                                       \
    case 13: FN<6, 7>(c, b, t, s); break;                                       \
    case 14: FN<7, 7>(c, b, t, s); break;                                       \
    case 15: FN<7, 8>(c, b, t, s); break;                                       \
    case 16: FN<8, 8>(c, b, t, s); break;                                       \
    case 17: FN<8, 9>(c, b, t, s); break;                                       \
    default: fail(PFA_ERR_INVALID_ARGUMENT, "unsupported poly_modulus_degree"); \
    }

void ntt_forward(const Ctx &c, const NttLaunch &a, hipStream_t s, bool allow_flow) {
    check_launch(c, a);
    const NttBatch b = make_batch(c, a);
    const NttTables t = tables(c);
    if (allow_flow && use_flow(c, b)) {
        flow<true>(c, b, t, s);
        return;
    }
    PFA_NTT_DISPATCH(fwd);
    PFA_HIP(hipGetLastError());
}

void ntt_inverse(const Ctx &c, const NttLaunch &a, hipStream_t s, bool allow_flow) {
    check_launch(c, a);
    const NttBatch b = make_batch(c, a);
    const NttTables t = tables(c);
    if (allow_flow && use_flow(c, b)) {
        flow<false>(c, b, t, s);
        return;
    }
    PFA_NTT_DISPATCH(inv);
    PFA_HIP(hipGetLastError());
}

void ntt_forward_rows(const Ctx &c, const NttLaunch &a, hipStream_t s) {
    check_launch(c, a);
    const NttBatch b = make_batch(c, a);
    const NttTables t = tables(c);
    PFA_NTT_DISPATCH(fwd_rows);
    PFA_HIP(hipGetLastError());
}

void ntt_inverse_cols(const Ctx &c, const NttLaunch &a, hipStream_t s) {
    check_launch(c, a);
    const NttBatch b = make_batch(c, a);
    const NttTables t = tables(c);
    PFA_NTT_DISPATCH(inv_cols);
    PFA_HIP(hipGetLastError());
}

// Streaming copy of n 16-byte words, each thread moving U words per round with
// nontemporal loads and stores: the achievable-bandwidth reference for the
// NTT's one-read-one-write traffic.
template <int U>
__global__ void __launch_bounds__(256) k_stream_copy(ulonglong2 *__restrict__ dst, const ulonglong2 *__restrict__ src,
                                                     uint64_t n) {
    const uint64_t stride = (uint64_t)gridDim.x * 256 * U;
    for (uint64_t base = (uint64_t)blockIdx.x * 256 * U + threadIdx.x; base < n; base += stride) {
        ulonglong2 v[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const uint64_t i = base + (uint64_t)u * 256;
            if (i < n) {
                v[u].x = __builtin_nontemporal_load(&src[i].x);
                v[u].y = __builtin_nontemporal_load(&src[i].y);
            }
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const uint64_t i = base + (uint64_t)u * 256;
            if (i < n) {
                __builtin_nontemporal_store(v[u].x, &dst[i].x);
                __builtin_nontemporal_store(v[u].y, &dst[i].y);
            }
        }
    }
}

bool xcd_round_robin(const Ctx &c) {
    constexpr uint32_t G = 1024;
    uint32_t *d = nullptr;
    PFA_HIP(hipMalloc((void **)&d, G * sizeof(uint32_t)));
    std::vector<uint32_t> h(G);
    hipLaunchKernelGGL(k_xcc_probe, dim3(G), dim3(64), 0, 0, d);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess) e = hipMemcpy(h.data(), d, G * sizeof(uint32_t), hipMemcpyDeviceToHost);
    (void)hipFree(d);
    PFA_HIP(e);
    // round-robin from the XCD of workgroup 0, which depends on earlier dispatches
    const uint32_t r = h[0];
    for (uint32_t i = 0; i < G; i++)
        if (h[i] != (i + r) % kXcds) return false;
    return true;
}

}  // namespace pfa

using namespace pfa;

extern "C" {

int pfa_ntt_forward(const pfa_context *ctx, uint64_t *inout, size_t M, size_t L, size_t start, void *stream) {
    return guarded([&] {
        const Ctx &c = *ctx_of(ctx);
        require(start + L <= c.QP, "limb range exceeds the context's primes");
        NttLaunch a{inout, inout, 0, 0, (uint32_t)M, (uint32_t)L};
        a.start = (uint32_t)start;
        ntt_forward(c, a, as_stream(stream));
    });
}

int pfa_stream_copy(uint64_t *dst, const uint64_t *src, size_t n, size_t workgroups, void *stream) {
    return guarded([&] {
        require(dst && src, "null data pointer");
        require(n % 2 == 0, "copy length must be a multiple of 2 words");
        require((reinterpret_cast<uintptr_t>(dst) & 15) == 0 && (reinterpret_cast<uintptr_t>(src) & 15) == 0,
                "copy buffers must be 16-byte aligned");
        const uint64_t n2 = n / 2;
        if (n2 == 0) return;
        const uint64_t need = (n2 + 256 * 4 - 1) / (256 * 4);
        const uint64_t grid = workgroups ? std::min<uint64_t>(workgroups, need) : need;
        hipLaunchKernelGGL(k_stream_copy<4>, dim3((uint32_t)grid), dim3(256), 0, as_stream(stream),
                           (ulonglong2 *)dst, (const ulonglong2 *)src, n2);
        PFA_HIP(hipGetLastError());
    });
}

int pfa_ntt_single_launch(const pfa_context *ctx, size_t M, size_t L, int *out) {
    return guarded([&] {
        const Ctx &c = *ctx_of(ctx);
        require(out != nullptr, "null argument");
        NttBatch b{};
        b.M = (uint32_t)M;
        b.L = (uint32_t)L;
        *out = M * L <= kFlowMaxJobs && use_flow(c, b) ? 1 : 0;
    });
}

int pfa_ntt_inverse(const pfa_context *ctx, uint64_t *inout, size_t M, size_t L, size_t start, void *stream) {
    return guarded([&] {
        const Ctx &c = *ctx_of(ctx);
        require(start + L <= c.QP, "limb range exceeds the context's primes");
        NttLaunch a{inout, inout, 0, 0, (uint32_t)M, (uint32_t)L};
        a.start = (uint32_t)start;
        ntt_inverse(c, a, as_stream(stream));
    });
}

}  // extern "C"
