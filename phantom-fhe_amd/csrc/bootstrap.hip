// Bootstrapping kernels.
//
// ModRaise (the raise step of mod_raise_inplace,
// src/bootstrap.cu): a ciphertext at the bottom of the chain (one prime q0,
// NTT form) is brought to coefficient form, each residue v is read as the
// centred integer (v - q0 when v >= floor(q0 / 2), as mod_raise_signed_tile_kernel
// does, src/bootstrap.cu:37-75), and that integer is reduced into every prime
// of the first data level, then the forward NTT runs over all of them.
// The result decrypts to m + q0 I over the full modulus, with I the small
// integer polynomial the rest of bootstrapping removes.
#include "internal.h"
#include "ntt_kernels.h"

namespace pfa {

namespace {

constexpr int kThreads = 256;

// in [size][N] residues mod q0 (coefficient form) -> out [size][L][N], table rows 0 .. L-1
__global__ void __launch_bounds__(kThreads)
k_lift_centered(const uint64_t *in, uint64_t *out, const uint64_t *mod, uint32_t L, uint32_t N) {
    const uint32_t l = blockIdx.y, p = blockIdx.z, n = blockIdx.x * kThreads + threadIdx.x;
    const uint64_t q0 = mod[0], q = mod[l];
    const uint64_t v = in[(size_t)p * N + n];
    uint64_t r;
    if (v < (q0 >> 1)) {
        r = v % q;
    } else {
        r = (q0 - v) % q;  // |v - q0|
        r = r ? q - r : 0;
    }
    st_stream(out + ((size_t)p * L + l) * N + n, r);
}

// out[k][l][n] = sum_t K_t in_t[k][l][n] (+ B on poly 0) mod q_l: the signed
// constants are reduced once per workgroup (its limb is blockIdx.y), the sum of
// up to kMaxTerms 128-bit products once per residue.
constexpr int kMaxTerms = 8;

struct LincombArgs {
    const uint64_t *in[kMaxTerms];
    uint32_t in_L[kMaxTerms];
    int64_t k[kMaxTerms];
    uint64_t b_lo, b_hi;  // signed 128-bit bias, two's complement
    uint32_t n, has_bias, L, N;
    uint32_t ct_size;     // polys per ciphertext: the bias goes to polys k with k mod ct_size = 0
};

__device__ __forceinline__ uint64_t signed_mod(int64_t v, uint64_t q) {
    const uint64_t m = v < 0 ? (uint64_t)0 - (uint64_t)v : (uint64_t)v;
    const uint64_t r = m % q;
    return v < 0 && r ? q - r : r;
}

// Each thread takes two adjacent residues (16-byte accesses) and requests
// every term's values before the first product: with the term loop rolled, the
// load of term t + 1 was issued only after term t's value had arrived (one
// load in flight per thread).

__global__ void __launch_bounds__(kThreads)
k_ct_lincomb(LincombArgs a, uint64_t *out, const uint64_t *mod, const ulonglong2 *ratio) {
    __shared__ uint64_t w[kMaxTerms + 1];
    const uint32_t l = blockIdx.y, k = blockIdx.z, n = (blockIdx.x * kThreads + threadIdx.x) * 2;
    const uint64_t q = mod[l];
    u64x2 v[kMaxTerms];
#pragma unroll
    for (int t = 0; t < kMaxTerms; t++)
        if (t < (int)a.n)
            v[t] = __builtin_nontemporal_load(
                reinterpret_cast<const u64x2 *>(a.in[t] + ((size_t)k * a.in_L[t] + l) * a.N + n));
    if (threadIdx.x < a.n) {
        w[threadIdx.x] = signed_mod(a.k[threadIdx.x], q);
    } else if (threadIdx.x == kMaxTerms) {
        uint64_t r = 0;
        if (a.has_bias && k % a.ct_size == 0) {
            const bool neg = (int64_t)a.b_hi < 0;
            U128 m{a.b_lo, a.b_hi};
            if (neg) {  // magnitude of the two's complement value
                m.lo = ~a.b_lo + 1;
                m.hi = ~a.b_hi + (m.lo == 0 ? 1 : 0);
            }
            r = barrett128(m, q, ratio[l].x, ratio[l].y);
            if (neg && r) r = q - r;
        }
        w[kMaxTerms] = r;
    }
    __syncthreads();
    U128 acc0{w[kMaxTerms], 0}, acc1{w[kMaxTerms], 0};
#pragma unroll
    for (int t = 0; t < kMaxTerms; t++)
        if (t < (int)a.n) {
            mac(acc0, w[t], v[t].x);
            mac(acc1, w[t], v[t].y);
        }
    u64x2 r;
    r.x = barrett128(acc0, q, ratio[l].x, ratio[l].y);
    r.y = barrett128(acc1, q, ratio[l].x, ratio[l].y);
    __builtin_nontemporal_store(r, reinterpret_cast<u64x2 *>(out + ((size_t)k * a.L + l) * a.N + n));
}

}  // namespace

}  // namespace pfa

using namespace pfa;

extern "C" {

int pfa_mod_raise(const pfa_context *ctx, const uint64_t *in, size_t size, uint64_t *out, void *stream) {
    return guarded([&] {
        const Ctx &c = *ctx_of(ctx);
        require(in && out, "null argument");
        require(size >= 1 && size <= 65535, "bad ciphertext size");
        const hipStream_t s = as_stream(stream);
        const uint32_t L = c.size_Ql(1);
        Scratch sc(c, s);
        uint64_t *coef = sc.alloc((size_t)size * c.N);
        NttLaunch inv{in, coef, (uint64_t)c.N, (uint64_t)c.N, (uint32_t)size, 1};
        ntt_inverse(c, inv, s);
        hipLaunchKernelGGL(k_lift_centered, dim3(c.N / kThreads, L, (uint32_t)size), dim3(kThreads), 0, s, coef, out,
                           c.mod, L, c.N);
        PFA_HIP(hipGetLastError());
        NttLaunch fw{out, out, (uint64_t)L * c.N, (uint64_t)L * c.N, (uint32_t)size, L};
        ntt_forward(c, fw, s);
    });
}

int pfa_ct_lincomb(const pfa_context *ctx, size_t L, size_t size, size_t ct_size, const uint64_t *const *ins,
                   const size_t *in_limbs, const int64_t *consts, size_t n, const uint64_t *bias, uint64_t *out,
                   void *stream) {
    return guarded([&] {
        const Ctx &c = *ctx_of(ctx);
        require(out && (n == 0 || (ins && in_limbs && consts)), "null argument");
        require(n <= (size_t)kMaxTerms, "at most 8 terms");
        require(L >= 1 && L <= c.QP, "limb count out of range");
        require(size >= 1 && size <= 65535, "bad ciphertext size");
        require(ct_size >= 1 && size % ct_size == 0, "size must be a multiple of the ciphertext size");
        LincombArgs a{};
        a.ct_size = (uint32_t)ct_size;
        for (size_t t = 0; t < n; t++) {
            require(ins[t] != nullptr, "null input");
            require(in_limbs[t] >= L && in_limbs[t] <= c.QP, "input has fewer limbs than the output");
            a.in[t] = ins[t];
            a.in_L[t] = (uint32_t)in_limbs[t];
            a.k[t] = consts[t];
        }
        a.n = (uint32_t)n;
        a.has_bias = bias != nullptr;
        if (bias) {
            a.b_lo = bias[0];
            a.b_hi = bias[1];
        }
        a.L = (uint32_t)L;
        a.N = c.N;
        require((reinterpret_cast<uintptr_t>(out) & 15) == 0, "output must be 16-byte aligned");
        for (size_t t = 0; t < n; t++) require((reinterpret_cast<uintptr_t>(ins[t]) & 15) == 0, "inputs must be 16-byte aligned");
        hipLaunchKernelGGL(k_ct_lincomb, dim3(c.N / (2 * kThreads), (uint32_t)L, (uint32_t)size), dim3(kThreads), 0,
                           as_stream(stream), a, out, c.mod, c.ratio);
        PFA_HIP(hipGetLastError());
    });
}

}  // extern "C"
