// Internal host-side declarations shared by the library's translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <array>
#include <initializer_list>
#include <map>
#include <mutex>
#include <stdexcept>
#include <string>
#include <thread>
#include <utility>
#include <vector>

#include "phantom_amd.h"

namespace pfa {

// ---------------------------------------------------------------- errors
// Exceptions carry the C-ABI status they map to; every extern "C" entry point
// catches them, records the message for pfa_last_error() and returns the code.
struct Error : std::runtime_error {
    int code;
    Error(int c, const std::string &m) : std::runtime_error(m), code(c) {}
};

[[noreturn]] inline void fail(int code, const std::string &msg) { throw Error(code, msg); }

inline void require(bool ok, const std::string &msg) {
    if (!ok) fail(PFA_ERR_INVALID_ARGUMENT, msg);
}

void hip_check(hipError_t e, const char *what);
#define PFA_HIP(x) ::pfa::hip_check((x), #x)

void set_last_error(const std::string &msg);
int handle_exception();

template <class F>
int guarded(F &&f) {
    try {
        f();
        return PFA_OK;
    } catch (...) {
        return handle_exception();
    }
}

inline hipStream_t as_stream(void *s) { return s ? (hipStream_t)s : hipStreamPerThread; }

// ---------------------------------------------------------------- host math
typedef unsigned __int128 u128;
inline uint64_t mulmod(uint64_t a, uint64_t b, uint64_t q) { return (uint64_t)((u128)a * b % q); }
uint64_t powmod(uint64_t a, uint64_t e, uint64_t q);
uint64_t invmod(uint64_t a, uint64_t q);  // q prime
inline uint64_t shoup_of(uint64_t w, uint64_t q) { return (uint64_t)(((u128)w << 64) / q); }
bool is_prime(uint64_t n);
uint64_t minimal_root(uint64_t degree, uint64_t q);
// Pair encoding of a constant w mod q for the NTT arithmetic policy of q
// (integer Shoup pair, or (double w, fl(w/q)) for q < 2^50).
ulonglong2 ntt_pair(uint64_t w, uint64_t q);
// Integer Shoup pair (w, floor(w 2^64/q)) for the elementwise kernels.
inline ulonglong2 shoup_pair(uint64_t w, uint64_t q) { return ulonglong2{w, shoup_of(w, q)}; }

// ---------------------------------------------------------------- context
// Constants of one chain level (chain index c >= 1, |Ql| = |Q| - c + 1),
// restating DRNSTool's per-level precompute (src/rns.cu:11-195).
struct Level {
    uint32_t Ql = 0, beta = 0;
    // ModUp: [(Q_part / q_i)^-1]_{q_i} per limb i < Ql, NTT-policy pairs
    ulonglong2 *modup_scale = nullptr;
    // ModUp: base-conversion matrix of digit b, [beta][alpha][QlP]:
    //   mat[b][i][r] = [Q_part_b / q_(b alpha + i)]_{p_r}   (p_r = prime of QlP row r)
    uint64_t *modup_mat = nullptr;
    // rescale: [q_last^-1]_{q_j} Shoup pairs, j < Ql - 1
    ulonglong2 *rescale_inv = nullptr;
    // fused path: modup_mat entries as NTT-policy pairs of the target prime,
    // [beta][alpha][QlP][2] = (m, [m 2^32]_{p_r}); rescale factor as NTT pairs
    ulonglong2 *modup_bc = nullptr;
    ulonglong2 *rescale_inv_p = nullptr;
    // fused ModDown + rescale, with q_l = this level's last prime:
    // INTT scales [1 + alpha] (unit pair of q_l, then the ModDown scales) and
    // [p_i^-1]_{q_l} for i < alpha (plain residues)
    ulonglong2 *mdr_scale = nullptr;
    uint64_t *mdr_glast = nullptr;
    // key-switch inner product: the QlP targets with the FP64-policy primes
    // first (in order), then the integer-policy ones
    uint32_t *ws_order = nullptr;
};

// Position -> item table of one k_bconv_cols launch shape: a permutation of
// `total` positions for a grid of `grid` workgroups (see lpt_schedule)
struct Sched {
    const uint32_t *table = nullptr;
    uint32_t grid = 0, total = 0;
};

// Work item w of a grouped launch: G groups of J items that read the same input
// tile.  A group's items all carry the same w mod 8, so in a grid whose size
// is a multiple of 8 they run on workgroups of one XCD (workgroups are dealt to
// the XCDs round-robin) and share its L2 copy of the input tile.
__host__ __device__ inline bool grouped_item(uint32_t w, uint32_t G, uint32_t J, uint32_t &g, uint32_t &j) {
    const uint32_t x = w & 7u, k = w >> 3;
    j = k % J;
    g = (k / J) * 8u + x;
    return g < G;
}

__host__ __device__ inline uint32_t grouped_total(uint32_t G, uint32_t J) { return ((G + 7u) / 8u) * 8u * J; }

// Static schedule of a persistent launch whose workgroup b runs positions b,
// b + R, b + 2R, ... < cost.size(): returns the position -> item permutation
// that gives the items, heaviest first, to the workgroup with the least
// assigned cost that still has a free position (longest-processing-time
// order), keeping every item on a workgroup congruent to it mod 8 (the same
// XCD when workgroups are dealt round-robin).  Empty when R is not a
// multiple of 8 or every workgroup has at most one position.
std::vector<uint32_t> lpt_schedule(const std::vector<uint8_t> &cost, uint32_t R);

// Device workspace of one (host thread, stream): chunks grown on demand and
// kept until the context is destroyed, handed out by a bump pointer.  Work on
// one stream runs in order, so memory released by a finished scope can be
// reused by the next call at once.  Keyed by thread as well as stream because
// hipStreamPerThread is one handle value shared by every thread.
struct Arena {
    struct Chunk {
        char *base;
        size_t cap, top;
    };
    std::vector<Chunk> chunks;
    // control blocks of the single-launch NTT on this stream (two, used in
    // turn; see FlowCtl in ntt_kernels.h), allocated on first use
    uint32_t *flow = nullptr;
    uint32_t flow_parity = 0;
    uint32_t flow_dirty[2] = {0, 0};  // jobs the last launch on each block used
    // arrival counters of the inner product's split items (k_inner_ws), zero
    // between launches (the last arrival clears its counter)
    uint32_t *ws_counter = nullptr;
};

struct Ctx {
    int device = 0;
    uint32_t N = 0, logN = 0;
    uint32_t QP = 0, P = 0, Q = 0;
    std::vector<uint64_t> moduli;  // Q primes then P primes
    std::vector<uint64_t> roots;   // minimal primitive 2N-th roots
    // device, all primes (rows of the QP table)
    uint64_t *mod = nullptr;        // [QP]
    ulonglong2 *ratio = nullptr;    // [QP] floor(2^128 / q) as (lo, hi)
    ulonglong2 *mont = nullptr;     // [QP] Montgomery constants (-q^-1 mod 2^64, 2^128 mod q)
    ulonglong2 *tw = nullptr;       // [QP][N]
    ulonglong2 *itw = nullptr;      // [QP][N]
    ulonglong2 *ninv = nullptr;     // [QP] NTT-policy pairs of N^-1
    ulonglong2 *small_fw = nullptr;  // [QP][256] psi^brv(j)
    ulonglong2 *small_inv = nullptr; // [QP][256] psi^-brv(j), no N^-1 fold
    ulonglong2 *rb_fw = nullptr;     // [QP][S2][N1] rows-pass stage bases tw[(N1 + k1) << g]
    ulonglong2 *rb_inv = nullptr;    // [QP][S2][N1] itw[(N1 + k1) << g]
    int n_cu = 256;                  // compute units of the device
    int ntt_wpc = 3;                 // resident workgroups per CU of the prefetching inverse rows pass
    int ntt_wpc_fwd = 4;             // the same for the passes without register prefetch
    uint64_t max_modulus = 0;        // the largest prime of the context
    uint32_t ws_slots = 0;           // resident inner-product workgroups assumed (0: from the occupancy API)
    // true when the device deals a launch's workgroups to its 8 XCDs
    // round-robin (probed once at context creation): the inner product splits
    // left-over items into digit chunks only then, and the single-launch NTT
    // is only enabled then
    bool xcd_rr = false;
    // single-launch NTT (ntt_kernels.h, opt-in): needs a device that deals
    // workgroups to 8 XCDs round-robin; used for batches of at least
    // flow_min_jobs limbs at N = 2^16
    bool ntt_flow = false;
    static constexpr int flow_wpc = 2;             // workgroups per CU
    uint32_t flow_window = 2;                      // jobs ahead of the second-pass front
    static constexpr uint32_t flow_min_jobs = 8;
    uint32_t flow_wait_ticks = 10000000;  // 100 ms at the 100 MHz s_memrealtime clock
    // Errors kernels record while they run, as a bit stored into the mapped
    // pinned host word err_host (1 a single-launch NTT's bounded wait expired,
    // 2 a single-launch NTT ended with tiles not transformed, 4 the digit
    // chunks of one inner-product item ran on different XCDs).  Reported by
    // check_device_errors, which reads the host word only (no device access),
    // at the entry of every C-ABI call that takes the context.
    uint32_t *err_host = nullptr;
    uint32_t *err_host_dev = nullptr;  // err_host's device address
    // ModDown (level independent): INTT scale [(P/p_j)^-1]_{p_j} (NTT pairs, [P]),
    // matrix [P/p_j]_{q_i} ([P][Q]), [P^-1]_{q_i} Shoup pairs ([Q])
    ulonglong2 *moddown_scale = nullptr;
    uint64_t *moddown_mat = nullptr;
    ulonglong2 *pinv = nullptr;
    // fused path: moddown_mat as NTT-policy pairs [P][Q][2] = (m, [m 2^32]_{q_i}),
    // (1, [2^32]_{q_i}) per Q prime [Q][2], [P^-1]_{q_i} as NTT-policy pairs [Q]
    ulonglong2 *moddown_bc = nullptr;
    ulonglong2 *unit_bc = nullptr;
    ulonglong2 *pinv_p = nullptr;
    // fused ModDown + rescale base conversion [1 + P][Q][2]: input 0 (the
    // rescale's last limb) with (1, [2^32]_{q_i}), input 1 + j with
    // ([p_j^-1]_{q_i}, [p_j^-1 2^32]_{q_i}), NTT-policy pairs
    ulonglong2 *mdr_bc = nullptr;
    // key construction: [P]_{q_i} Shoup pairs over all QP rows (0 on P rows)
    ulonglong2 *pmodq = nullptr;
    uint32_t *slot_perm = nullptr;   // [N/2] CKKS slot j -> DFT index (5^j mod 2N - 1) / 4
    ulonglong2 *crt_inv = nullptr;   // [Q][Q] q_i^-1 mod q_j (i < j) as Shoup pairs: the decoder's Garner composition
    std::vector<Level> levels;  // index = chain index (0 unused)
    std::vector<void *> allocations;
    mutable std::mutex arena_mu;
    mutable std::map<std::pair<std::thread::id, hipStream_t>, Arena *> arenas;
    // Pinned host staging for small host-to-device uploads (pointer tables):
    // a copy from pageable memory would make the host wait for the stream's
    // earlier work; from pinned memory it is queued like a kernel.  Slots are
    // reused round-robin once their previous copy has completed (its event).
    static constexpr size_t kStageSlots = 64, kStageSlotBytes = 64 << 10;
    char *stage = nullptr;                       // hipHostMalloc'd, kStageSlots * kStageSlotBytes
    hipEvent_t stage_ev[kStageSlots] = {};
    mutable std::mutex stage_mu;
    mutable size_t stage_next = 0;
    // work schedules of the base-conversion and epilogue launches by (kind,
    // shape), built on first use (modup_schedule, epi_schedule); their device
    // tables are freed with the context
    mutable std::mutex sched_mu;
    mutable std::map<std::array<uint32_t, 4>, Sched> scheds;
    mutable std::vector<void *> sched_allocs;

    uint32_t size_Ql(uint32_t chain) const { return Q - (chain - 1); }
    const Level &level(uint32_t chain) const {
        require(chain >= 1 && chain <= Q, "chain index out of range");
        return levels[chain];
    }
    // physical table row of position r of the QlP basis (Ql primes, then P primes)
    uint32_t qlp_row(uint32_t Ql, uint32_t r) const { return r < Ql ? r : Q + (r - Ql); }
    template <class T>
    T *upload(const std::vector<T> &v);
};

template <class T>
T *Ctx::upload(const std::vector<T> &v) {
    void *p = nullptr;
    PFA_HIP(hipMalloc(&p, (v.empty() ? 1 : v.size()) * sizeof(T)));
    allocations.push_back(p);
    if (!v.empty()) PFA_HIP(hipMemcpy(p, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice));
    return (T *)p;
}

// The schedule of the ModUp base conversion of `batch` key switches at chain
// index `chain` (k_bconv_cols over batch x beta digits x column tiles x QlP
// targets), built and uploaded on first use: a synchronous upload, so the
// first key switch of a shape must not run under stream capture (the first
// call of a shape also grows the workspace).  Batches above 64 get none.
Sched modup_schedule(const Ctx &c, uint32_t chain, uint32_t batch);
// The schedule of a k_epi_rows launch over M polys x J target limbs (the
// level's first J primes) x `tiles` row tiles on `grid` workgroups, built
// and uploaded on first use like modup_schedule; none when every workgroup
// has at most one item.
Sched epi_schedule(const Ctx &c, uint32_t J, uint32_t M, uint32_t tiles, uint32_t grid);

Ctx *ctx_of(const pfa_context *c);
// Throws PFA_ERR_RUNTIME (and clears the record) if a kernel of this context
// recorded an error on the device since the last check.  Kernels record it in
// mapped host memory, so the check sees it once the kernel has run; it makes
// no HIP call, so it is safe under stream capture.  ctx_of runs it, i.e. every
// C-ABI call that takes a context checks before it launches anything.
void check_device_errors(const Ctx &c);
// The calling thread's workspace for stream s (its single-launch NTT control
// blocks live there).
Arena &arena_for(const Ctx &c, hipStream_t s);
void encoder_init(Ctx &c);

// RAII scope over the calling thread's workspace for stream s: alloc() hands
// out 256-byte-aligned device memory, all of it released when the scope ends.
// Copies n bytes from host memory to device memory dst in stream order
// without waiting for the stream (pinned staging; larger copies than a slot
// fall back to a plain asynchronous copy).
void upload_async(const Ctx &c, void *dst, const void *src, size_t n, hipStream_t s);
// Host tables packed into one block of sc (each part at a 16-byte aligned
// offset) and uploaded with one copy on s; dev[i] receives part i's address.
struct HostPart {
    const void *src;
    size_t bytes;
};
class Scratch;
void upload_parts(const Ctx &c, Scratch &sc, hipStream_t s, std::initializer_list<HostPart> parts, void **dev);

class Scratch {
  public:
    Scratch(const Ctx &c, hipStream_t s);
    ~Scratch();
    Scratch(const Scratch &) = delete;
    Scratch &operator=(const Scratch &) = delete;
    template <class T = uint64_t>
    T *alloc(size_t elems) {
        return (T *)alloc_bytes(elems * sizeof(T));
    }

  private:
    void *alloc_bytes(size_t bytes);
    Arena &a_;
    std::vector<size_t> marks_;
};

// ---------------------------------------------------------------- launchers
// NTT over M polys x L limbs; see NttBatch in ntt_kernels.h for the fields.
struct NttLaunch {
    const uint64_t *src;
    uint64_t *dst;
    uint64_t sstride, dstride;  // poly strides (elements); 0 -> L * N
    uint32_t M, L;
    uint32_t start = 0, split = 0xffffffffu, split_base = 0;
    uint32_t ex_lo = 0, ex_step = 0, ex_len = 0, ex_cap = 0;
    const ulonglong2 *scale = nullptr;
};
// allow_flow false keeps the transform on the two-launch path, which needs no
// workspace (the single-launch path takes control blocks from it)
void ntt_forward(const Ctx &c, const NttLaunch &a, hipStream_t s, bool allow_flow = true);
void ntt_inverse(const Ctx &c, const NttLaunch &a, hipStream_t s, bool allow_flow = true);
// The inverse's columns pass alone: a.src holds the output of its rows pass
// (fused_tensor_rows), a.dst receives the canonical coefficients.
void ntt_inverse_cols(const Ctx &c, const NttLaunch &a, hipStream_t s);
// the forward NTT's rows pass alone, over a columns pass's output in a.src
void ntt_forward_rows(const Ctx &c, const NttLaunch &a, hipStream_t s);
// True when the device deals a launch's workgroups to 8 XCDs round-robin
// (workgroup w on XCD (w + r) mod 8 for some r), which the single-launch NTT is
// built for; runs a probe kernel.
bool xcd_round_robin(const Ctx &c);

// Fused key-switching / rescale pipelines (fused_ks.hip).
// c2 [Ql][N] (NTT form) -> cx [2][QlP][N]: ModUp then the inner product with key.
// With batch > 1, member i reads c2 + i c2_stride and writes cx + i cx_stride
// (default 2 QlP N), all with the same key.
// With fold, limb Ql - 1 of output k of member i is written as
// (fold->base_k + i stride)[Ql - 1] + cx_k[Ql - 1] [P^-1]: the input
// fused_moddown_rescale expects.
struct KsFold {
    const uint64_t *base0 = nullptr, *base1 = nullptr;
    uint64_t stride = 0;
};
// With key_table (a device array of batch key pointers), member i uses its own key.
// With c2_mid ([batch][Ql][N], from fused_tensor_rows), the ModUp's INTT runs
// its columns pass only, on c2_mid.
void fused_modup_inner(const Ctx &c, uint32_t chain, const uint64_t *c2, const uint64_t *key, uint64_t *cx,
                       hipStream_t s, uint32_t batch = 1, uint64_t c2_stride = 0, uint64_t cx_stride = 0,
                       const KsFold *fold = nullptr, const uint64_t *const *key_table = nullptr,
                       const uint64_t *c2_mid = nullptr);
// ModUp of c2 (Ql limbs, NTT form) into out [beta][QlP][N] in NTT form, by the
// fused base conversion + columns pass and then the rows pass; each digit's
// own limbs are not written (they are c2's).
void fused_modup_ntt(const Ctx &c, uint32_t chain, const uint64_t *c2, uint64_t *out, hipStream_t s);
// The tensor product of count ciphertext pairs (as op_tensor: member i reads
// a, b at + i in_stride, writes d0, d1 at + i d_stride, d2 at + i d2_stride)
// with the first pass of the key switch's INTT(d2) fused in: mid [count][Ql][N]
// receives the inverse rows pass over d2, the input fused_modup_inner takes as
// c2_mid.  N = 2^10 .. 2^16.
void fused_tensor_rows(const Ctx &c, uint32_t chain, const uint64_t *a, const uint64_t *b, uint64_t *d0,
                       uint64_t *d1, uint64_t *d2, uint64_t *mid, hipStream_t s, uint32_t count,
                       uint64_t in_stride, uint64_t d_stride, uint64_t d2_stride);
// The rotation input of B ciphertexts (src[i] at src + i src_stride): dst
// [B][2][Ql][N] = both polys through the Galois permutation of element elt (or
// elts[i], a device table), plus add0 on poly 0 when given (B = 1), and mid
// [B][Ql][N] = the inverse rows pass over dst's poly 1, the input
// fused_modup_inner takes as c2_mid.  N = 2^10 .. 2^16.
void galois_rows(const Ctx &c, uint32_t chain, const uint64_t *src, uint64_t src_stride, uint32_t B, uint32_t elt,
                 const uint32_t *elts, const uint64_t *add0, uint64_t *dst, uint64_t *mid, hipStream_t s);
// cx [2][QlP][N] from fused_modup_inner with a fold over base -> out [2][Ql-1][N]
// = rescale(base + ModDown(cx)), bit-identical to fused_moddown then fused_rescale.
// With count > 1: cx [count][2][QlP][N], member i's bases at + i base_stride,
// out [count][2][Ql-1][N].
void fused_moddown_rescale(const Ctx &c, uint32_t chain, const uint64_t *cx, const uint64_t *base0,
                           const uint64_t *base1, uint64_t *out, hipStream_t s, uint32_t count = 1,
                           uint64_t base_stride = 0);
// cx [M][QlP][N] -> out [M][Ql][N] = base + ModDown(cx): poly 2i + k adds
// base_k + i base_stride; the bases may alias out's polys or be null.
void fused_moddown(const Ctx &c, uint32_t chain, const uint64_t *cx, uint32_t M, uint64_t *out,
                   const uint64_t *base0, const uint64_t *base1, hipStream_t s, uint64_t base_stride = 0);
// in [size][Ql][N] -> out [size][Ql-1][N]: floor division by the level's last prime.
void fused_rescale(const Ctx &c, uint32_t chain, const uint64_t *in, uint32_t size, uint64_t *out, hipStream_t s);
// The same with the caller's buffers for the last limb's coefficients (last,
// size N) and the base conversion's intermediate (inter, size (Ql - 1) N; may
// be out itself: the epilogue rewrites each tile of it in place); allocates
// nothing when allow_flow is false (no single-launch NTT control blocks, no
// epilogue work schedule).
void fused_rescale_with(const Ctx &c, uint32_t chain, const uint64_t *in, uint32_t size, uint64_t *out,
                        uint64_t *last, uint64_t *inter, hipStream_t s, bool allow_flow);
// Allocation-free entry points (noalloc.hip): takes the address of this
// device's static scratch array; called once per device, with it current.
void noalloc_init(int device);

}  // namespace pfa
