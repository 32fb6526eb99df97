// Allocation-free rescale for callers that cannot allocate device memory
// (code under HIP graph capture, serving loops or harnesses that forbid
// hipMalloc).  The reference has no counterpart: its rescale_to_next allocates
// its temporaries stream-ordered (src/evaluate.cu:1413-1464).
//
// pfa_rescale takes two temporaries from the calling thread's workspace (grown
// with hipMalloc on first use): the last limb of each input poly in coefficient
// form, and the base conversion's columns-pass intermediate.  Here the
// intermediate is formed in the output buffer itself (the epilogue reads each
// tile of it and writes the same tile), and the coefficients go to `scratch`,
// one static array per device, shared by every call on that device until the
// process ends.  Calls that overlap in time on one device (different streams
// or threads) race on it; calls on one stream are ordered.  Nothing in it has
// to start at zero: a call overwrites what it reads.
#include <mutex>

#include "internal.h"

namespace pfa {

namespace {

// size x N residues: 4 polys at N = 2^17, 8 at N = 2^16 (4 MiB)
constexpr size_t kNoAllocWords = (size_t)4 << 17;

static __device__ __align__(256) uint64_t scratch[kNoAllocWords];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
uint64_t *g_scratch[kMaxDevices] = {};  // scratch's device address, per device

uint64_t *scratch_of(int device) {
    std::lock_guard<std::mutex> lock(g_mu);
    return device >= 0 && device < kMaxDevices ? g_scratch[device] : nullptr;
}

}  // namespace

// Called by pfa_context_create with `device` current.  The array's name in
// host code is only a stand-in for the symbol; its device address (one per
// device) is what kernels and copies must use.
void noalloc_init(int device) {
    require(device >= 0 && device < kMaxDevices, "device index out of range");
    std::lock_guard<std::mutex> lock(g_mu);
    if (g_scratch[device]) return;
    void *p = nullptr;
    PFA_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    g_scratch[device] = (uint64_t *)p;
}

}  // namespace pfa

using namespace pfa;

extern "C" {

int pfa_rescale_noalloc(const pfa_context *ctx, size_t chain_index, const uint64_t *in, size_t size, uint64_t *out,
                        void *stream) {
    return guarded([&] {
        const Ctx &c = *ctx_of(ctx);
        require(in && out, "null argument");
        require(chain_index >= 1 && chain_index <= c.Q, "chain index out of range (key level 0 is not a data level)");
        const uint32_t L = c.level((uint32_t)chain_index).Ql;
        require(L >= 2, "cannot rescale at the last level");
        require(size >= 1, "bad ciphertext size");
        require(size * c.N <= kNoAllocWords,
                "pfa_rescale_noalloc: size x N = " + std::to_string(size * c.N) + " residues exceeds its scratch of " +
                    std::to_string(kNoAllocWords) + " (use pfa_rescale)");
        // the intermediate is formed in out before in is read
        const uintptr_t i0 = (uintptr_t)in, i1 = i0 + (uintptr_t)size * L * c.N * 8;
        const uintptr_t o0 = (uintptr_t)out, o1 = o0 + (uintptr_t)size * (L - 1) * c.N * 8;
        require(o1 <= i0 || i1 <= o0, "pfa_rescale_noalloc: input and output buffers overlap");
        uint64_t *last = scratch_of(c.device);
        if (!last) fail(PFA_ERR_LOGIC, "pfa_rescale_noalloc: the device's scratch was not set up");
        fused_rescale_with(c, (uint32_t)chain_index, in, (uint32_t)size, out, last, out, as_stream(stream), false);
    });
}

}  // extern "C"
