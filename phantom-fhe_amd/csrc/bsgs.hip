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

// Pointer list of the accumulation: a device table, or (no table) an
// arithmetic progression base + i * stride, which is how contiguous batches of
// plaintexts and outputs arrive; neither needs a host-to-device copy.
template <class P>
struct PtrList {
    P *const *table;
    P *base;
    uint64_t stride;  // elements
    __device__ __forceinline__ P *operator[](size_t i) const { return table ? table[i] : base + i * stride; }
};

constexpr uint32_t kInlineBabies = 64;

struct MacArgs {
    PtrList<const uint64_t> pt;  // [G M] plaintexts, [Ql][N] each (NTT form)
    PtrList<uint64_t> out;       // [G] ciphertexts, [2][Ql][N] each
    const uint64_t *const *baby_table;          // [M] ciphertexts [2][Ql][N], when M > kInlineBabies
    const uint64_t *baby_inline[kInlineBabies];  // the same, by value, when M <= kInlineBabies
    uint32_t M, G, Ql, N;
    __device__ __forceinline__ const uint64_t *baby(uint32_t b) const {
        return baby_table ? baby_table[b] : baby_inline[b];
    }
};

// A work item covers kSpan consecutive residues of one limb (kSpan / 256 per
// thread, 256 apart), so every plaintext is read in 8 KiB runs.
// FP64 policy: each product is within 0.875 q (|x y / q| < q < 2^50), so four
// of them on top of a reduced sum stay below 4 q < 2^53; integer policy: 128-bit
// sums of at most eight products below q^2 < 2^122, then one Barrett reduction.
constexpr uint32_t kSpan = 1024;
constexpr int kPer = kSpan / kThreads;

__global__ void __launch_bounds__(kThreads)
k_bsgs_mac(MacArgs a, const uint64_t *mod, const ulonglong2 *ratio) {
    const uint32_t T = a.N / kSpan;  // items per limb and giant
    const uint32_t groups = a.Ql * T;
    const uint32_t total = grouped_total(groups, a.G);
    for (uint32_t w = blockIdx.x; w < total; w += gridDim.x) {
        uint32_t grp, g;
        if (!grouped_item(w, groups, a.G, grp, g)) continue;
        const uint32_t j = grp / T, tile = grp % T;
        const size_t off0 = (size_t)j * a.N + tile * kSpan + threadIdx.x;
        const size_t off1 = off0 + (size_t)a.Ql * a.N;
        const uint64_t q = mod[j];
        const size_t pt0 = (size_t)g * a.M;
        uint64_t *o = a.out[g];
        if (q < kF64PrimeBound) {
            const ArithF64 ar(q);
            double acc0[kPer], acc1[kPer];
#pragma unroll
            for (int e = 0; e < kPer; e++) acc0[e] = acc1[e] = 0.0;
            for (uint32_t b = 0; b < a.M; b++) {
                const uint64_t *p = a.pt[pt0 + b] + off0;
                const uint64_t *c = a.baby(b);
                double x[kPer], y0[kPer], y1[kPer];
#pragma unroll
                for (int e = 0; e < kPer; e++) {
                    x[e] = ar.load(ld_stream(p + e * kThreads));
                    y0[e] = ar.load(c[off0 + e * kThreads]);
                    y1[e] = ar.load(c[off1 + e * kThreads]);
                }
#pragma unroll
                for (int e = 0; e < kPer; e++) {
                    const double xq = x[e] * ar.qinv;
                    acc0[e] += ar.mulw(y0[e], x[e], xq);
                    acc1[e] += ar.mulw(y1[e], x[e], xq);
                }
                if ((b & 3u) == 3u) {
#pragma unroll
                    for (int e = 0; e < kPer; e++) {
                        ar.reduce(acc0[e]);
                        ar.reduce(acc1[e]);
                    }
                }
            }
#pragma unroll
            for (int e = 0; e < kPer; e++) {
                st_stream(o + off0 + e * kThreads, ar.store(acc0[e]));
                st_stream(o + off1 + e * kThreads, ar.store(acc1[e]));
            }
        } else {
            const ulonglong2 r = ratio[j];
            U128 s0[kPer], s1[kPer];
#pragma unroll
            for (int e = 0; e < kPer; e++) s0[e] = s1[e] = U128{0, 0};
            for (uint32_t b = 0; b < a.M; b++) {
                const uint64_t *p = a.pt[pt0 + b] + off0;
                const uint64_t *c = a.baby(b);
#pragma unroll
                for (int e = 0; e < kPer; e++) {
                    const uint64_t x = ld_stream(p + e * kThreads);
                    mac(s0[e], x, c[off0 + e * kThreads]);
                    mac(s1[e], x, c[off1 + e * kThreads]);
                }
                if ((b & 7u) == 7u) {
#pragma unroll
                    for (int e = 0; e < kPer; e++) {
                        s0[e] = U128{barrett128(s0[e], q, r.x, r.y), 0};
                        s1[e] = U128{barrett128(s1[e], q, r.x, r.y), 0};
                    }
                }
            }
#pragma unroll
            for (int e = 0; e < kPer; e++) {
                st_stream(o + off0 + e * kThreads, barrett128(s0[e], q, r.x, r.y));
                st_stream(o + off1 + e * kThreads, barrett128(s1[e], q, r.x, r.y));
            }
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

// Both polys of a ciphertext through the Galois permutation of NTT slots
// (apply_galois_ntt_permutation, src/galois.cu:11-18):
//   dst[k][l][i] = src[k][l][pi(i)]  (+ add0[l][i] for k = 0 when add0 is given).
__global__ void __launch_bounds__(kThreads)
k_galois_ct(const uint64_t *src, uint64_t *dst, const uint64_t *add0, const uint64_t *mod, uint32_t elt, uint32_t L,
            uint32_t N, uint32_t logN) {
    const uint32_t l = blockIdx.y, k = blockIdx.z, n = blockIdx.x * kThreads + threadIdx.x;
    const size_t row = ((size_t)k * L + l) * N;
    uint64_t v = src[row + galois_perm(elt, n, logN)];
    if (k == 0 && add0) v = add_mod(v, add0[(size_t)l * N + n], mod[l]);
    st_stream(dst + row + n, v);
}

// out = rotate(src) (+ add): the Galois permutation of both polys, then the
// key switch of the permuted c1 whose ModDown epilogue adds the permuted c0
// (and add[0]) to poly 0 and add[1] to poly 1 -- apply_galois_with_ksk
// (src/evaluate.cu:1607-1656) followed by add_inplace, with the same residues.
// out must not alias src; add[1] may alias out's poly 1.
void rotate_into(const Ctx &c, uint32_t chain, const uint64_t *src, uint32_t elt, const uint64_t *key,
                 const uint64_t *add, uint64_t *out, hipStream_t s) {
    const uint32_t Ql = c.size_Ql(chain), QlP = Ql + c.P;
    const size_t LN = (size_t)Ql * c.N;
    Scratch sc(c, s);
    uint64_t *t = sc.alloc(2 * LN);
    hipLaunchKernelGGL(k_galois_ct, dim3(c.N / kThreads, Ql, 2), dim3(kThreads), 0, s, src, t, add, c.mod, elt, Ql,
                       c.N, c.logN);
    PFA_HIP(hipGetLastError());
    uint64_t *cx = sc.alloc((size_t)2 * QlP * c.N);
    fused_modup_inner(c, chain, t + LN, key, cx, s);
    fused_moddown(c, chain, cx, 2, out, t, add ? add + LN : nullptr, s);
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
        MacArgs a{};
        a.M = (uint32_t)M;
        a.G = (uint32_t)G;
        a.Ql = Ql;
        a.N = c.N;
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
        if (progression((const void *const *)pts, M * G, st)) {
            a.pt = PtrList<const uint64_t>{nullptr, pts[0], st};
        } else {
            const uint64_t **t = sc.alloc<const uint64_t *>(M * G);
            PFA_HIP(hipMemcpyAsync(t, pts, M * G * sizeof(void *), hipMemcpyHostToDevice, s));
            a.pt = PtrList<const uint64_t>{t, nullptr, 0};
        }
        if (progression((const void *const *)out, G, st)) {
            a.out = PtrList<uint64_t>{nullptr, out[0], st};
        } else {
            uint64_t **t = sc.alloc<uint64_t *>(G);
            PFA_HIP(hipMemcpyAsync(t, out, G * sizeof(void *), hipMemcpyHostToDevice, s));
            a.out = PtrList<uint64_t>{t, nullptr, 0};
        }
        if (M <= kInlineBabies) {
            for (size_t i = 0; i < M; i++) a.baby_inline[i] = babies[i];
        } else {
            const uint64_t **t = sc.alloc<const uint64_t *>(M);
            PFA_HIP(hipMemcpyAsync(t, babies, M * sizeof(void *), hipMemcpyHostToDevice, s));
            a.baby_table = t;
        }
        const uint32_t total = grouped_total(Ql * (c.N / kSpan), (uint32_t)G);
        const uint32_t cap = (uint32_t)c.n_cu * 8u;
        hipLaunchKernelGGL(k_bsgs_mac, dim3(total < cap ? total : cap), dim3(kThreads), 0, s, a, c.mod, c.ratio);
        PFA_HIP(hipGetLastError());
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
        const size_t ct_elems = (size_t)2 * c.size_Ql(chain) * c.N;
        // babies[b] = rotate(babies[b - msb(b)], msb(b)); babies[0] = ct, babies[b] = out[b - 1]
        for (size_t b = 1; b < M; b++) {
            uint32_t k = 0;
            while ((size_t)2 << k <= b) k++;
            const size_t rem = b - ((size_t)1 << k);
            const uint64_t *src = rem ? out + (rem - 1) * ct_elems : ct;
            rotate_into(c, chain, src, elts[k], keys[k], nullptr, out + (b - 1) * ct_elems, s);
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
            rotate_into(c, chain, pg + ct_elems, elt, key, pg, pg, s);
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
