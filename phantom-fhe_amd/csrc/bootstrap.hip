// ModRaise for CKKS bootstrapping (the raise step of mod_raise_inplace,
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

}  // extern "C"
