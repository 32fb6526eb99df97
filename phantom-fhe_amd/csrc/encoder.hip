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
// precision, one launch per stage.  Decoding composes each coefficient from
// the first two RNS limbs (Garner), exact for |m_k| < q0 q1 / 2 (~2^109 with a
// 60-bit q0), and centres it.
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

// z_k = w_k zeta^-k / M; coefficients -> RNS residues of the L first primes.
__global__ void k_enc_round(const double2 *w, uint64_t *out, const uint64_t *mod, uint32_t L, uint32_t N,
                            double scale_over_m, uint32_t *overflow) {
    const uint32_t M = N / 2;
    for (uint32_t k = blockIdx.x * blockDim.x + threadIdx.x; k < M; k += gridDim.x * blockDim.x) {
        double s, c;
        sincospi(-(double)k / (double)N, &s, &c);  // zeta^-k = exp(-i pi k / N)
        const double2 v = w[k];
        const double re = (v.x * c - v.y * s) * scale_over_m;
        const double im = (v.x * s + v.y * c) * scale_over_m;
        const double r[2] = {rint(re), rint(im)};
        for (int h = 0; h < 2; h++) {
            const double x = r[h];
            if (!(fabs(x) < 4611686018427387904.0)) {  // 2^62 (also catches NaN)
                atomicOr(overflow, 1u);
                continue;
            }
            const bool neg = x < 0;
            const uint64_t a = (uint64_t)fabs(x);
            for (uint32_t l = 0; l < L; l++) {
                const uint64_t q = mod[l];
                uint64_t t = a % q;
                if (neg && t) t = q - t;
                out[(size_t)l * N + k + h * M] = t;
            }
        }
    }
}

// z_k = w_k zeta^-k / M -> the rounded integer coefficients themselves (the
// reference's level-independent single-chain plaintext, src/single_chain_plaintext.cu:93-150).
__global__ void k_enc_round_signed(const double2 *w, int64_t *out, uint32_t N, double scale_over_m,
                                   uint32_t *overflow) {
    const uint32_t M = N / 2;
    for (uint32_t k = blockIdx.x * blockDim.x + threadIdx.x; k < M; k += gridDim.x * blockDim.x) {
        double s, c;
        sincospi(-(double)k / (double)N, &s, &c);
        const double2 v = w[k];
        const double r[2] = {rint((v.x * c - v.y * s) * scale_over_m), rint((v.x * s + v.y * c) * scale_over_m)};
        for (int h = 0; h < 2; h++) {
            if (!(fabs(r[h]) < 4611686018427387904.0)) {  // 2^62 (also catches NaN)
                atomicOr(overflow, 1u);
                out[k + h * M] = 0;
            } else {
                out[k + h * M] = (int64_t)r[h];
            }
        }
    }
}

// Coefficient-form limbs -> twisted complex vector w_k = z_k zeta^k, z_k = (m_k + i m_(k+M)) / scale.
__global__ void k_dec_compose(const uint64_t *coef, double2 *w, uint64_t q0, uint64_t q1, uint64_t q0inv_mod_q1,
                              ulonglong2 r1, uint32_t L, uint32_t N, double inv_scale) {
    const uint32_t M = N / 2;
    // Q = q0 q1 and floor(Q / 2) as 128-bit (hi, lo)
    const uint64_t Qlo = q0 * q1, Qhi = mulhi64(q0, q1);
    const uint64_t Hlo = (Qlo >> 1) | (Qhi << 63), Hhi = Qhi >> 1;
    for (uint32_t k = blockIdx.x * blockDim.x + threadIdx.x; k < M; k += gridDim.x * blockDim.x) {
        double v[2];
        for (int h = 0; h < 2; h++) {
            const uint32_t i = k + h * M;
            const uint64_t c0 = coef[i];
            if (L == 1) {
                v[h] = c0 > q0 / 2 ? -(double)(q0 - c0) : (double)c0;
            } else {
                // Garner: x = c0 + q0 * ((c1 - c0) q0^-1 mod q1), in [0, q0 q1)
                const uint64_t c1 = coef[(size_t)N + i];
                const uint64_t d = sub_mod(c1, c0 >= q1 ? c0 % q1 : c0, q1);
                const uint64_t t = barrett128(U128{d * q0inv_mod_q1, mulhi64(d, q0inv_mod_q1)}, q1, r1.x, r1.y);
                uint64_t xlo = q0 * t, xhi = mulhi64(q0, t);
                xlo += c0;
                xhi += xlo < c0 ? 1 : 0;
                const bool upper = xhi > Hhi || (xhi == Hhi && xlo > Hlo);
                if (upper) {  // x - Q, negative
                    const uint64_t nlo = Qlo - xlo;
                    const uint64_t nhi = Qhi - xhi - (Qlo < xlo ? 1 : 0);
                    v[h] = -((double)nhi * 18446744073709551616.0 + (double)nlo);
                } else {
                    v[h] = (double)xhi * 18446744073709551616.0 + (double)xlo;
                }
            }
        }
        double s, c;
        sincospi((double)k / (double)N, &s, &c);  // zeta^k
        const double re = v[0] * inv_scale, im = v[1] * inv_scale;
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
        require(scale > 0 && std::isfinite(scale), "scale out of bounds");
        const hipStream_t s = as_stream(stream);
        Scratch sc(c, s);
        double2 *buf = sc.alloc<double2>(2 * (size_t)M);
        uint32_t *flag = sc.alloc<uint32_t>(1);
        hipLaunchKernelGGL(k_zero_flag, dim3(1), dim3(1), 0, s, flag);
        hipLaunchKernelGGL(k_enc_scatter, ew_grid(M), dim3(kThreads), 0, s, (const double2 *)values,
                           (uint32_t)n_values, buf, c.slot_perm, M);
        double2 *w = fft(buf, buf + M, M, -1.0, s);
        hipLaunchKernelGGL(k_enc_round, ew_grid(M), dim3(kThreads), 0, s, w, out, c.mod, (uint32_t)L, c.N,
                           scale / (double)M, flag);
        PFA_HIP(hipGetLastError());
        uint32_t h_flag = 0;
        PFA_HIP(hipMemcpyAsync(&h_flag, flag, sizeof(uint32_t), hipMemcpyDeviceToHost, s));
        PFA_HIP(hipStreamSynchronize(s));
        require(h_flag == 0, "encoded values are too large");
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
        require(scale > 0 && std::isfinite(scale), "scale out of bounds");
        const hipStream_t s = as_stream(stream);
        Scratch sc(c, s);
        double2 *buf = sc.alloc<double2>(2 * (size_t)M);
        uint32_t *flag = sc.alloc<uint32_t>(1);
        hipLaunchKernelGGL(k_zero_flag, dim3(1), dim3(1), 0, s, flag);
        hipLaunchKernelGGL(k_enc_scatter, ew_grid(M), dim3(kThreads), 0, s, (const double2 *)values,
                           (uint32_t)n_values, buf, c.slot_perm, M);
        double2 *w = fft(buf, buf + M, M, -1.0, s);
        hipLaunchKernelGGL(k_enc_round_signed, ew_grid(M), dim3(kThreads), 0, s, w, coeffs, c.N, scale / (double)M,
                           flag);
        PFA_HIP(hipGetLastError());
        uint32_t h_flag = 0;
        PFA_HIP(hipMemcpyAsync(&h_flag, flag, sizeof(uint32_t), hipMemcpyDeviceToHost, s));
        PFA_HIP(hipStreamSynchronize(s));
        require(h_flag == 0, "encoded values are too large");
    });
}

int pfa_ckks_decode(const pfa_context *ctx, const uint64_t *in, size_t L, double scale, double *values, void *stream) {
    return guarded([&] {
        const Ctx &c = *ctx_of(ctx);
        require(in && values, "null argument");
        require(L >= 1 && L <= c.Q, "plaintext limb count out of range");
        require(scale > 0 && std::isfinite(scale), "scale out of bounds");
        const hipStream_t s = as_stream(stream);
        const uint32_t M = c.N / 2;
        const uint32_t Lc = L >= 2 ? 2 : 1;
        Scratch sc(c, s);
        uint64_t *coef = sc.alloc((size_t)Lc * c.N);
        double2 *buf = sc.alloc<double2>(2 * (size_t)M);
        NttLaunch inv{in, coef, 0, 0, 1, Lc};
        ntt_inverse(c, inv, s);
        const uint64_t q0 = c.moduli[0], q1 = c.moduli[Lc > 1 ? 1 : 0];
        const uint64_t q0inv = Lc > 1 ? invmod(q0 % q1, q1) : 0;
        const ulonglong2 r1{(uint64_t)((~(u128)0 / q1)), (uint64_t)((~(u128)0 / q1) >> 64)};
        hipLaunchKernelGGL(k_dec_compose, ew_grid(M), dim3(kThreads), 0, s, coef, buf, q0, q1, q0inv, r1, Lc, c.N,
                           1.0 / scale);
        double2 *W = fft(buf, buf + M, M, 1.0, s);
        hipLaunchKernelGGL(k_dec_gather, ew_grid(M), dim3(kThreads), 0, s, W, (double2 *)values, c.slot_perm, M);
        PFA_HIP(hipGetLastError());
    });
}

}  // extern "C"
