// BSGS matrix-vector product support: the giant-step accumulation of
// bsgs_apply_giants_with_babies (src/bsgs.cu:51-96, :272-296), for every giant
// in one launch, and the batched expansion of level-independent plaintexts
// (signed coefficients, light_pt_expand_per_tower_kernel, src/bsgs.cu:16-23).
//
// Accumulation: out[g][k][j] = sum_{b < M} pt[g M + b][j] * baby[b][k][j]
// (mod q_j) for giant g, ciphertext poly k in {0, 1} and limb j.  The reference
// runs one launch per giant, reading all M babies each time; here a work item
// is (limb tile, giant) and the items of one limb tile are grouped on one XCD,
// so a tile of the babies is read from HBM once and then from that XCD's L2
// for every giant.  Results are canonical residues, equal to the reference's
// per-step Barrett sums.
#include "internal.h"
#include "ntt_kernels.h"

namespace pfa {

namespace {

constexpr int kThreads = 256;

struct MacArgs {
    const uint64_t *const *pt;    // [G M] plaintexts, [Ql][N] each (NTT form)
    const uint64_t *const *baby;  // [M] ciphertexts, [2][Ql][N] each (NTT form)
    uint64_t *const *out;         // [G] ciphertexts, [2][Ql][N] each
    uint32_t M, G, Ql, N;
};

// FP64 policy: each product is within 0.875 q (|x y / q| < q < 2^50), so four
// of them on top of a reduced sum stay below 4 q < 2^53; integer policy: 128-bit
// sums of at most eight products below q^2 < 2^122, then one Barrett reduction.
__global__ void __launch_bounds__(kThreads)
k_bsgs_mac(MacArgs a, const uint64_t *mod, const ulonglong2 *ratio) {
    const uint32_t T = a.N / kThreads;  // tiles per limb
    const uint32_t groups = a.Ql * T;
    const uint32_t total = grouped_total(groups, a.G);
    for (uint32_t w = blockIdx.x; w < total; w += gridDim.x) {
        uint32_t grp, g;
        if (!grouped_item(w, groups, a.G, grp, g)) continue;
        const uint32_t j = grp / T, tile = grp % T;
        const size_t off0 = (size_t)j * a.N + tile * kThreads + threadIdx.x;
        const size_t off1 = off0 + (size_t)a.Ql * a.N;
        const uint64_t q = mod[j];
        const uint64_t *const *pt = a.pt + (size_t)g * a.M;
        uint64_t *o = a.out[g];
        if (q < kF64PrimeBound) {
            const ArithF64 ar(q);
            double acc0 = 0.0, acc1 = 0.0;
            for (uint32_t b = 0; b < a.M; b++) {
                const double x = ar.load(ld_stream(pt[b] + off0));
                const double xq = x * ar.qinv;
                const uint64_t *c = a.baby[b];
                acc0 += ar.mulw(ar.load(c[off0]), x, xq);
                acc1 += ar.mulw(ar.load(c[off1]), x, xq);
                if ((b & 3u) == 3u) {
                    ar.reduce(acc0);
                    ar.reduce(acc1);
                }
            }
            st_stream(o + off0, ar.store(acc0));
            st_stream(o + off1, ar.store(acc1));
        } else {
            const ulonglong2 r = ratio[j];
            U128 s0{0, 0}, s1{0, 0};
            for (uint32_t b = 0; b < a.M; b++) {
                const uint64_t x = ld_stream(pt[b] + off0);
                const uint64_t *c = a.baby[b];
                mac(s0, x, c[off0]);
                mac(s1, x, c[off1]);
                if ((b & 7u) == 7u) {
                    s0 = U128{barrett128(s0, q, r.x, r.y), 0};
                    s1 = U128{barrett128(s1, q, r.x, r.y), 0};
                }
            }
            st_stream(o + off0, barrett128(s0, q, r.x, r.y));
            st_stream(o + off1, barrett128(s1, q, r.x, r.y));
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

}  // namespace

}  // namespace pfa

using namespace pfa;

extern "C" {

int pfa_bsgs_mac(const pfa_context *ctx, size_t chain_index, const uint64_t *const *pts,
                 const uint64_t *const *babies, size_t M, size_t G, uint64_t *const *out, void *stream) {
    return guarded([&] {
        const Ctx &c = *ctx_of(ctx);
        require(pts && babies && out, "null argument");
        require(M >= 1 && G >= 1, "need at least one baby step and one giant step");
        require(M * G < (1u << 24), "too many plaintexts");
        if (chain_index < 1 || chain_index > c.Q) fail(PFA_ERR_INVALID_ARGUMENT, "chain index out of range");
        for (size_t i = 0; i < M * G; i++) require(pts[i] != nullptr, "null plaintext pointer");
        for (size_t i = 0; i < M; i++) require(babies[i] != nullptr, "null ciphertext pointer");
        for (size_t i = 0; i < G; i++) require(out[i] != nullptr, "null output pointer");
        const hipStream_t s = as_stream(stream);
        const uint32_t Ql = c.size_Ql((uint32_t)chain_index);
        Scratch sc(c, s);
        const uint64_t **dpt = sc.alloc<const uint64_t *>(M * G);
        const uint64_t **dbaby = sc.alloc<const uint64_t *>(M);
        uint64_t **dout = sc.alloc<uint64_t *>(G);
        PFA_HIP(hipMemcpyAsync(dpt, pts, M * G * sizeof(void *), hipMemcpyHostToDevice, s));
        PFA_HIP(hipMemcpyAsync(dbaby, babies, M * sizeof(void *), hipMemcpyHostToDevice, s));
        PFA_HIP(hipMemcpyAsync(dout, out, G * sizeof(void *), hipMemcpyHostToDevice, s));
        const MacArgs a{dpt, dbaby, dout, (uint32_t)M, (uint32_t)G, Ql, c.N};
        const uint32_t total = grouped_total(Ql * (c.N / kThreads), (uint32_t)G);
        const uint32_t cap = (uint32_t)c.n_cu * 8u;
        hipLaunchKernelGGL(k_bsgs_mac, dim3(total < cap ? total : cap), dim3(kThreads), 0, s, a, c.mod, c.ratio);
        PFA_HIP(hipGetLastError());
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
