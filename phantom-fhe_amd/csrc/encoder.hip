// CKKS encoder / decoder on the GPU (PhantomCKKSEncoder, src/ckks.cu:17-190;
// special FFT, src/fft.cu).
//
// Slot j of a real-coefficient plaintext m(X) mod X^N + 1 is m(zeta^(5^j)),
// zeta = exp(2 pi i / 2N), j < N/2.  Because zeta^(5^j N/2) = i, with
// z_k = m_k + i m_(k+N/2) (k < N/2) that is sum_k z_k zeta^(k 5^j), and since
// {5^j mod 2N} = {1 + 4t}, it is a length-N/2 DFT of the twisted vector
// w_k = z_k zeta^k read at index t_j = (5^j mod 2N - 1) / 4:
//   decode: w = z * zeta^k, W = DFT+(w), slot_j = W[t_j]
//   encode: W[t_j] = slot_j, w = DFT-(W) / (N/2), z = w * zeta^-k,
//           m_k = round(scale Re z_k), m_(k+N/2) = round(scale Im z_k)
// (the reference's encode packs coefficients the same way,
// src/rns_base.cu:49-72).  The DFT is a radix-2 Stockham FFT in double
// precision, one launch per stage.  A rounded coefficient is reduced into each
// prime exactly at any size a double holds (m 2^e with 2^e mod q by squaring,
// where the reference splits it into 64-bit words, src/rns_base.cu:49-170).
// Decoding composes each coefficient from all of the plaintext's limbs
// (Garner's mixed radix, then centred against floor(Q/2)) as the reference's
// compose_array does (src/rns_base.cu:173-253), so it is exact for any
// |m_k| < Q / 2.
#include <cmath>

#include "internal.h"
#include "modarith.h"

namespace pfa {

namespace {

constexpr int kThreads = 256;

__global__ void k_enc_scatter(const double2 *values, uint32_t n_values, double2 *W, const uint32_t *perm,
                              uint32_t M) {
    for (uint32_t j = blockIdx.x * blockDim.x + threadIdx.x; j < M; j += gridDim.x * blockDim.x)
        W[perm[j]] = j < n_values ? values[j] : double2{0.0, 0.0};
}

__global__ void k_dec_gather(const double2 *W, double2 *values, const uint32_t *perm, uint32_t M) {
    for (uint32_t j = blockIdx.x * blockDim.x + threadIdx.x; j < M; j += gridDim.x * blockDim.x)
        values[j] = W[perm[j]];
}

// One Stockham radix-2 stage of a length-M DFT with kernel exp(sign i 2 pi jk / M);
// Ns = current sub-transform length.
__global__ void k_fft_stage(const double2 *in, double2 *out, uint32_t M, uint32_t Ns, double sign) {
    const uint32_t half = M / 2;
    for (uint32_t j = blockIdx.x * blockDim.x + threadIdx.x; j < half; j += gridDim.x * blockDim.x) {
        const uint32_t k = j & (Ns - 1);
        double s, c;
        sincospi(sign * (double)k / (double)Ns, &s, &c);
        const double2 a = in[j], b0 = in[j + half];
        const double2 b{b0.x * c - b0.y * s, b0.x * s + b0.y * c};
        const uint32_t base = (j - k) * 2 + k;
        out[base] = double2{a.x + b.x, a.y + b.y};
        out[base + Ns] = double2{a.x - b.x, a.y - b.y};
    }
}

// a b mod q for any a, b < 2^64 (ratio = floor(2^128 / q))
__device__ __forceinline__ uint64_t mulmod_any(uint64_t a, uint64_t b, uint64_t q, ulonglong2 rt) {
    return barrett128(mul_wide(a, b), q, rt.x, rt.y);
}

// x mod q for a double x >= 0 that holds an integer: below 2^62 directly,
// above it as m 2^e (53-bit m, e >= 10) with 2^e mod q by squaring.
__device__ __forceinline__ uint64_t dbl_int_mod(double x, uint64_t q, ulonglong2 rt) {
    if (x < 4611686018427387904.0) return barrett128(U128{(uint64_t)x, 0}, q, rt.x, rt.y);  // 2^62
    const uint64_t bits = (uint64_t)__double_as_longlong(x);
    uint32_t e = (uint32_t)((bits >> 52) & 0x7ff) - 1075u;
    const uint64_t m = (bits & ((1ull << 52) - 1)) | (1ull << 52);
    uint64_t p = 1, b = 2;  // primes here are at least 2N + 1
    for (; e; e >>= 1) {
        if (e & 1u) p = mulmod_any(p, b, q, rt);
        b = mulmod_any(b, b, q, rt);
    }
    return mulmod_any(barrett128(U128{m, 0}, q, rt.x, rt.y), p, q, rt);
}

// The reference's size check (src/ckks.cu:112-126): ceil(log2(max(|v|, 1))) + 1
// bits, exact from the binary exponent; not finite: ~0u.
__device__ __forceinline__ uint32_t coeff_bits(double v) {
    const double a = fabs(v);
    if (!(a < __builtin_huge_val())) return ~0u;
    if (a <= 1.0) return 1;
    int ex;
    const double m = frexp(a, &ex);  // a = m 2^ex, m in [0.5, 1)
    return (uint32_t)(m > 0.5 ? ex : ex - 1) + 1;
}

// z_k = w_k zeta^-k / M; coefficients -> RNS residues of the L first primes.
// bits receives the largest coeff_bits of the unrounded coefficients.
__global__ void k_enc_round(const double2 *w, uint64_t *out, const uint64_t *mod, const ulonglong2 *ratio,
                            uint32_t L, uint32_t N, double scale_over_m, uint32_t *bits) {
    const uint32_t M = N / 2;
    uint32_t mb = 1;
    for (uint32_t k = blockIdx.x * blockDim.x + threadIdx.x; k < M; k += gridDim.x * blockDim.x) {
        double s, c;
        sincospi(-(double)k / (double)N, &s, &c);  // zeta^-k = exp(-i pi k / N)
        const double2 v = w[k];
        const double re = (v.x * c - v.y * s) * scale_over_m;
        const double im = (v.x * s + v.y * c) * scale_over_m;
        const double u[2] = {re, im};
        for (int h = 0; h < 2; h++) {
            const uint32_t b = coeff_bits(u[h]);
            mb = b > mb ? b : mb;
            const double x = rint(u[h]);
            const bool neg = x < 0;
            const double a = b == ~0u ? 0.0 : fabs(x);
            for (uint32_t l = 0; l < L; l++) {
                const uint64_t q = mod[l];
                uint64_t t = dbl_int_mod(a, q, ratio[l]);
                if (neg && t) t = q - t;
                out[(size_t)l * N + k + h * M] = t;
            }
        }
    }
    atomicMax(bits, mb);
}

// z_k = w_k zeta^-k / M -> the reference's level-independent single-chain
// coefficients (src/single_chain_plaintext.cu:93-150): the rounded
// coefficient's residue mod q0, centred into (-q0/2, q0/2].
__global__ void k_enc_round_signed(const double2 *w, int64_t *out, uint32_t N, double scale_over_m, uint64_t q0,
                                   ulonglong2 r0, uint32_t *bits) {
    const uint32_t M = N / 2;
    uint32_t mb = 1;
    for (uint32_t k = blockIdx.x * blockDim.x + threadIdx.x; k < M; k += gridDim.x * blockDim.x) {
        double s, c;
        sincospi(-(double)k / (double)N, &s, &c);
        const double2 v = w[k];
        const double u[2] = {(v.x * c - v.y * s) * scale_over_m, (v.x * s + v.y * c) * scale_over_m};
        for (int h = 0; h < 2; h++) {
            const uint32_t b = coeff_bits(u[h]);
            mb = b > mb ? b : mb;
            const double x = rint(u[h]);
            uint64_t t = dbl_int_mod(b == ~0u ? 0.0 : fabs(x), q0, r0);
            if (x < 0 && t) t = q0 - t;
            out[k + h * M] = t > q0 / 2 ? -(int64_t)(q0 - t) : (int64_t)t;
        }
    }
    atomicMax(bits, mb);
}

// Coefficient i of the L coefficient-form limbs as a double times inv_scale,
// centred (compose_array, src/rns_base.cu:173-253): Garner's mixed-radix
// digits v_j (x = sum_j v_j prod_{i<j} q_i, each v_j < q_j) are written over
// the limbs in place, x is compared with floor(Q/2) digit by digit from the top
// (the digits of (Q - 1) / 2 by long division in the same radix), and the
// value is x or -(Q - x).  inv[i][j] = q_i^-1 mod q_j as Shoup pairs.
__device__ double compose_one(uint64_t *coef, size_t i, const uint64_t *mod, const ulonglong2 *ratio,
                              const ulonglong2 *inv, uint32_t Q, uint32_t L, uint32_t N, double inv_scale) {
    for (uint32_t j = 1; j < L; j++) {
        const uint64_t q = mod[j];
        const ulonglong2 rt = ratio[j];
        uint64_t t = coef[(size_t)j * N + i];
        for (uint32_t l = 0; l < j; l++) {
            const uint64_t v = barrett128(U128{coef[(size_t)l * N + i], 0}, q, rt.x, rt.y);
            const ulonglong2 f = inv[(size_t)l * Q + j];
            t = shoup(sub_mod(t, v, q), f.x, f.y, q);
        }
        coef[(size_t)j * N + i] = t;
    }
    int cmp = 0;
    uint64_t r = 0;
    for (uint32_t j = L; j-- > 0;) {
        const uint64_t q = mod[j], v = coef[(size_t)j * N + i];
        const uint64_t d = r * q + (q - 1);  // < 2 q
        const uint64_t h = d >> 1;
        r = d & 1;
        if (cmp == 0) cmp = v > h ? 1 : (v < h ? -1 : 0);
    }
    // x, or Q - x = (Q - 1 - x) + 1 with digits q_j - 1 - v_j and a carry
    const bool neg = cmp > 0;
    double res = 0.0, wj = inv_scale;
    uint64_t carry = 1;
    for (uint32_t j = 0; j < L; j++) {
        const uint64_t q = mod[j], v = coef[(size_t)j * N + i];
        uint64_t dj = v;
        if (neg) {
            dj = q - 1 - v + carry;
            carry = dj == q ? 1 : 0;
            dj = carry ? 0 : dj;
        }
        if (dj) res += (double)dj * wj;  // zero digits skipped: wj may have overflowed
        wj *= (double)q;
    }
    return neg ? -res : res;
}

// Coefficient-form limbs -> twisted complex vector w_k = z_k zeta^k, z_k = (m_k + i m_(k+M)) / scale.
__global__ void k_dec_compose(uint64_t *coef, double2 *w, const uint64_t *mod, const ulonglong2 *ratio,
                              const ulonglong2 *inv, uint32_t Q, uint32_t L, uint32_t N, double inv_scale) {
    const uint32_t M = N / 2;
    for (uint32_t k = blockIdx.x * blockDim.x + threadIdx.x; k < M; k += gridDim.x * blockDim.x) {
        const double re = compose_one(coef, k, mod, ratio, inv, Q, L, N, inv_scale);
        const double im = compose_one(coef, k + M, mod, ratio, inv, Q, L, N, inv_scale);
        double s, c;
        sincospi((double)k / (double)N, &s, &c);  // zeta^k
        w[k] = double2{re * c - im * s, re * s + im * c};
    }
}

__global__ void k_zero_flag(uint32_t *p) { *p = 0; }

inline dim3 ew_grid(uint32_t n) { return dim3(std::min<uint32_t>((n + kThreads - 1) / kThreads, 4096)); }

// In-place (ping-pong) length-M FFT; returns the buffer holding the result.
double2 *fft(double2 *a, double2 *b, uint32_t M, double sign, hipStream_t s) {
    for (uint32_t Ns = 1; Ns < M; Ns <<= 1) {
        hipLaunchKernelGGL(k_fft_stage, ew_grid(M / 2), dim3(kThreads), 0, s, a, b, M, Ns, sign);
        std::swap(a, b);
    }
    return a;
}

}  // namespace

void encoder_init(Ctx &c) {
    const uint32_t M = c.N / 2, m2 = 2 * c.N;
    std::vector<uint32_t> perm(M);
    uint64_t p = 1;
    for (uint32_t j = 0; j < M; j++) {
        perm[j] = (uint32_t)((p - 1) / 4);
        p = (p * 5) % m2;
    }
    c.slot_perm = c.upload(perm);
    std::vector<ulonglong2> inv((size_t)c.Q * c.Q, ulonglong2{0, 0});
    for (uint32_t i = 0; i < c.Q; i++)
        for (uint32_t j = i + 1; j < c.Q; j++) {
            const uint64_t q = c.moduli[j], v = invmod(c.moduli[i] % q, q);
            inv[(size_t)i * c.Q + j] = ulonglong2{v, shoup_of(v, q)};
        }
    c.crt_inv = c.upload(inv);
}

// Bit length of q_0 q_1 ... q_(L-1) (the reference's total_coeff_modulus_bit_count
// of the level with L primes), by exact multi-word products.
static uint32_t total_bits(const Ctx &c, uint32_t L) {
    std::vector<uint64_t> p{1};
    for (uint32_t i = 0; i < L; i++) {
        u128 carry = 0;
        for (uint64_t &w : p) {
            const u128 t = (u128)w * c.moduli[i] + carry;
            w = (uint64_t)t;
            carry = t >> 64;
        }
        if (carry) p.push_back((uint64_t)carry);
    }
    return 64 * (uint32_t)(p.size() - 1) + (64 - (uint32_t)__builtin_clzll(p.back()));
}

static ulonglong2 host_ratio(uint64_t q) { return ulonglong2{(uint64_t)(~(u128)0 / q), (uint64_t)((~(u128)0 / q) >> 64)}; }

// The reference's scale bound (src/ckks.cu:87-89 encode, :148-151 decode).
static void check_scale(double scale, uint32_t tb, int extra) {
    require(scale > 0 && std::isfinite(scale) && (int)std::log2(scale) + extra < (int)tb, "scale out of bounds");
}

}  // namespace pfa

using namespace pfa;

extern "C" {

int pfa_ckks_encode(const pfa_context *ctx, const double *values, size_t n_values, double scale, uint64_t *out,
                    size_t L, void *stream) {
    return guarded([&] {
        const Ctx &c = *ctx_of(ctx);
        require(out && (values || n_values == 0), "null argument");
        const uint32_t M = c.N / 2;
        require(n_values >= 1, "Input vector is empty");
        require(n_values <= M, "Input vector exceeds max slots");
        require(L >= 1 && L <= c.Q, "plaintext limb count out of range");
        const uint32_t tb = total_bits(c, (uint32_t)L);
        check_scale(scale, tb, 1);
        const hipStream_t s = as_stream(stream);
        Scratch sc(c, s);
        double2 *buf = sc.alloc<double2>(2 * (size_t)M);
        uint32_t *flag = sc.alloc<uint32_t>(1);
        hipLaunchKernelGGL(k_zero_flag, dim3(1), dim3(1), 0, s, flag);
        hipLaunchKernelGGL(k_enc_scatter, ew_grid(M), dim3(kThreads), 0, s, (const double2 *)values,
                           (uint32_t)n_values, buf, c.slot_perm, M);
        double2 *w = fft(buf, buf + M, M, -1.0, s);
        hipLaunchKernelGGL(k_enc_round, ew_grid(M), dim3(kThreads), 0, s, w, out, c.mod, c.ratio, (uint32_t)L, c.N,
                           scale / (double)M, flag);
        PFA_HIP(hipGetLastError());
        uint32_t h_flag = 0;
        PFA_HIP(hipMemcpyAsync(&h_flag, flag, sizeof(uint32_t), hipMemcpyDeviceToHost, s));
        PFA_HIP(hipStreamSynchronize(s));
        require(h_flag < tb, "encoded values are too large");  // src/ckks.cu:122-126
        NttLaunch fw{out, out, 0, 0, 1, (uint32_t)L};
        ntt_forward(c, fw, s);
    });
}

int pfa_ckks_encode_coeffs(const pfa_context *ctx, const double *values, size_t n_values, double scale,
                           int64_t *coeffs, void *stream) {
    return guarded([&] {
        const Ctx &c = *ctx_of(ctx);
        require(coeffs && (values || n_values == 0), "null argument");
        const uint32_t M = c.N / 2;
        require(n_values >= 1, "Input vector is empty");
        require(n_values <= M, "Input vector exceeds max slots");
        // encoded at chain index 1 (all of Q), then reduced mod q0 and centred
        const uint32_t tb = total_bits(c, c.Q);
        check_scale(scale, tb, 1);
        const hipStream_t s = as_stream(stream);
        Scratch sc(c, s);
        double2 *buf = sc.alloc<double2>(2 * (size_t)M);
        uint32_t *flag = sc.alloc<uint32_t>(1);
        hipLaunchKernelGGL(k_zero_flag, dim3(1), dim3(1), 0, s, flag);
        hipLaunchKernelGGL(k_enc_scatter, ew_grid(M), dim3(kThreads), 0, s, (const double2 *)values,
                           (uint32_t)n_values, buf, c.slot_perm, M);
        double2 *w = fft(buf, buf + M, M, -1.0, s);
        hipLaunchKernelGGL(k_enc_round_signed, ew_grid(M), dim3(kThreads), 0, s, w, coeffs, c.N, scale / (double)M,
                           c.moduli[0], host_ratio(c.moduli[0]), flag);
        PFA_HIP(hipGetLastError());
        uint32_t h_flag = 0;
        PFA_HIP(hipMemcpyAsync(&h_flag, flag, sizeof(uint32_t), hipMemcpyDeviceToHost, s));
        PFA_HIP(hipStreamSynchronize(s));
        require(h_flag < tb, "encoded values are too large");
    });
}

int pfa_ckks_decode(const pfa_context *ctx, const uint64_t *in, size_t L, double scale, double *values, void *stream) {
    return guarded([&] {
        const Ctx &c = *ctx_of(ctx);
        require(in && values, "null argument");
        require(L >= 1 && L <= c.Q, "plaintext limb count out of range");
        check_scale(scale, total_bits(c, (uint32_t)L), 0);
        const hipStream_t s = as_stream(stream);
        const uint32_t M = c.N / 2;
        Scratch sc(c, s);
        uint64_t *coef = sc.alloc((size_t)L * c.N);
        double2 *buf = sc.alloc<double2>(2 * (size_t)M);
        NttLaunch inv{in, coef, 0, 0, 1, (uint32_t)L};
        ntt_inverse(c, inv, s);
        hipLaunchKernelGGL(k_dec_compose, ew_grid(M), dim3(kThreads), 0, s, coef, buf, c.mod, c.ratio, c.crt_inv, c.Q,
                           (uint32_t)L, c.N, 1.0 / scale);
        double2 *W = fft(buf, buf + M, M, 1.0, s);
        hipLaunchKernelGGL(k_dec_gather, ew_grid(M), dim3(kThreads), 0, s, W, (double2 *)values, c.slot_perm, M);
        PFA_HIP(hipGetLastError());
    });
}

}  // extern "C"
