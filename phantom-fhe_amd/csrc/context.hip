// Context construction: moduli, NTT tables and per-level RNS constants.
//
// Host precompute restated from the mathematics of the reference's
// src/host/{modulus,numth,ntt,rns}.cu and src/rns.cu:11-195; all tables are
// uploaded once to HBM and are read-only afterwards.
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <mutex>

#include "internal.h"
#include "modarith.h"

namespace pfa {

// ---------------------------------------------------------------- errors
static thread_local std::string g_last_error;

void set_last_error(const std::string &msg) { g_last_error = msg; }

void hip_check(hipError_t e, const char *what) {
    if (e != hipSuccess) fail(PFA_ERR_RUNTIME, std::string(what) + ": " + hipGetErrorString(e));
}

int handle_exception() {
    try {
        throw;
    } catch (const Error &e) {
        set_last_error(e.what());
        return e.code;
    } catch (const std::invalid_argument &e) {
        set_last_error(e.what());
        return PFA_ERR_INVALID_ARGUMENT;
    } catch (const std::logic_error &e) {
        set_last_error(e.what());
        return PFA_ERR_LOGIC;
    } catch (const std::exception &e) {
        set_last_error(e.what());
        return PFA_ERR_RUNTIME;
    } catch (...) {
        set_last_error("unknown error");
        return PFA_ERR_RUNTIME;
    }
}

// ---------------------------------------------------------------- host math
uint64_t powmod(uint64_t a, uint64_t e, uint64_t q) {
    uint64_t r = 1 % q;
    a %= q;
    for (; e; e >>= 1) {
        if (e & 1) r = mulmod(r, a, q);
        a = mulmod(a, a, q);
    }
    return r;
}

uint64_t invmod(uint64_t a, uint64_t q) {
    a %= q;
    if (a == 0) fail(PFA_ERR_INVALID_ARGUMENT, "value not invertible");
    return powmod(a, q - 2, q);
}

// Deterministic Miller-Rabin: the first twelve primes as bases decide every
// n < 3.3e24 (the reference decides the same question with 40 random rounds,
// src/host/numth.cu:129-205).
bool is_prime(uint64_t n) {
    static const uint64_t bases[] = {2, 3, 5, 7, 11, 13, 17, 19, 23, 29, 31, 37};
    if (n < 2) return false;
    for (uint64_t p : bases) {
        if (n % p == 0) return n == p;
    }
    uint64_t d = n - 1;
    int s = 0;
    while (!(d & 1)) {
        d >>= 1;
        ++s;
    }
    for (uint64_t a : bases) {
        uint64_t x = powmod(a, d, n);
        if (x == 1 || x == n - 1) continue;
        bool composite = true;
        for (int i = 1; i < s && composite; ++i) {
            x = mulmod(x, x, n);
            if (x == n - 1) composite = false;
        }
        if (composite) return false;
    }
    return true;
}

// Smallest primitive degree-th root of unity mod q (try_minimal_primitive_root,
// src/host/numth.cu:309-331).  The primitive roots are the odd powers of any
// one of them; a first one comes from x^((q-1)/degree) for the smallest x whose
// power has order exactly degree.
uint64_t minimal_root(uint64_t degree, uint64_t q) {
    if ((q - 1) % degree) fail(PFA_ERR_INVALID_ARGUMENT, "prime is not congruent to 1 mod 2N");
    const uint64_t cof = (q - 1) / degree;
    uint64_t g = 0;
    for (uint64_t x = 2; x < q && !g; ++x) {
        uint64_t c = powmod(x, cof, q);
        if (powmod(c, degree / 2, q) == q - 1) g = c;
    }
    if (!g) fail(PFA_ERR_INVALID_ARGUMENT, "no primitive root");
    const uint64_t g2 = mulmod(g, g, q);
    uint64_t best = g;
    for (uint64_t k = 1, cur = g; k < degree; k += 2, cur = mulmod(cur, g2, q)) best = std::min(best, cur);
    return best;
}

ulonglong2 ntt_pair(uint64_t w, uint64_t q) {
    if (q < (1ULL << 50)) {
        double wd = (double)w, wq = (double)w / (double)q;
        uint64_t a, b;
        std::memcpy(&a, &wd, 8);
        std::memcpy(&b, &wq, 8);
        return ulonglong2{a, b};
    }
    return shoup_pair(w, q);
}

static uint32_t bitrev(uint32_t x, int bits) {
    uint32_t r = 0;
    for (int i = 0; i < bits; ++i) r |= ((x >> i) & 1u) << (bits - 1 - i);
    return r;
}

// ---------------------------------------------------------------- primes
// CoeffModulus::Create (src/host/modulus.cu:80-111): for each bit size b the
// candidates are 2^b - 2N + 1, 2^b - 4N + 1, ... (q = 1 mod 2N, q > 2^(b-1));
// the k requests of size b receive the k largest such primes, smallest first.
static void create_coeff_modulus(uint64_t N, const int *bits, size_t count, uint64_t *out) {
    // the reference's limits (src/host/modulus.cu:80-94, include/host/defines.h:11-24)
    require(N >= 2 && N <= 131072 && (N & (N - 1)) == 0, "poly_modulus_degree is invalid");
    require(count <= 64, "bit_sizes is invalid: at most 64 moduli");
    for (size_t i = 0; i < count; ++i) require(bits[i] >= 2 && bits[i] <= 60, "bit size must be in [2, 60]");
    std::vector<int> sizes(bits, bits + count);
    std::sort(sizes.begin(), sizes.end());
    sizes.erase(std::unique(sizes.begin(), sizes.end()), sizes.end());
    for (int b : sizes) {
        size_t want = std::count(bits, bits + count, b);
        std::vector<uint64_t> found;
        const uint64_t step = 2 * N, lower = 1ULL << (b - 1);
        uint64_t v = (1ULL << b) - step + 1;
        while (found.size() < want) {
            if (v <= lower) fail(PFA_ERR_LOGIC, "failed to find enough qualifying primes");
            if (is_prime(v)) found.push_back(v);
            v -= step;
        }
        std::reverse(found.begin(), found.end());  // smallest first
        size_t k = 0;
        for (size_t i = 0; i < count; ++i)
            if (bits[i] == b) out[i] = found[k++];
    }
}

// ---------------------------------------------------------------- context
static uint64_t two32_mod(uint64_t q) { return (uint64_t)(((u128)1 << 32) % q); }

// Second factor pair of a base-conversion entry m for target q: FP64 policy,
// the pair of m 2^32 mod q (the high half of a wide input); integer policy,
// m 2^64 mod q (the factor of the Montgomery-accumulated conversion).
static ulonglong2 bconv_pair1(uint64_t m, uint64_t q) {
    if (q < kF64PrimeBound) return ntt_pair(mulmod(m, two32_mod(q), q), q);
    const uint64_t r64 = (uint64_t)((((u128)1 << 64) - 1) % q + 1) % q;  // 2^64 mod q
    return ulonglong2{mulmod(m, r64, q), 0};
}

static uint64_t prod_mod(const uint64_t *m, size_t n, size_t skip, uint64_t p) {
    uint64_t r = 1 % p;
    for (size_t k = 0; k < n; ++k)
        if (k != skip) r = mulmod(r, m[k] % p, p);
    return r;
}

// Argument checks of PhantomContext construction, done before any device call.
static void validate(uint64_t N, const uint64_t *moduli, size_t QP, size_t P) {
    require(N >= 1024 && N <= (1u << 17) && (N & (N - 1)) == 0, "poly_modulus_degree must be 2^10 .. 2^17");
    require(QP >= 2 && P >= 1 && P < QP, "need at least one data prime and one special prime");
    for (size_t i = 0; i < QP; ++i) {
        uint64_t q = moduli[i];
        require(q < (1ULL << 61) && q % (2 * N) == 1 && is_prime(q), "moduli must be primes = 1 mod 2N below 2^61");
        for (size_t j = 0; j < i; ++j) require(moduli[j] != q, "moduli must be distinct");
    }
}

static void build(Ctx &c, uint64_t N, const uint64_t *moduli, size_t QP, size_t P) {
    c.N = (uint32_t)N;
    c.logN = 0;
    while ((1u << c.logN) < c.N) ++c.logN;
    c.QP = (uint32_t)QP;
    c.P = (uint32_t)P;
    c.Q = (uint32_t)(QP - P);
    c.moduli.assign(moduli, moduli + QP);

    // NTT tables (src/host/ntt.cu:11-56): tw[brv(i)] = psi^i, itw[brv(i)] = psi^-i,
    // itw[1] *= N^-1.
    // rows-pass geometry of the NTT kernels: N = N1 * N2 with S1 = min(8, logN / 2)
    const uint32_t S1 = c.logN / 2 > 8 ? 8 : c.logN / 2, S2 = c.logN - S1, N1 = 1u << S1;
    std::vector<ulonglong2> tw(QP * N), itw(QP * N), ninv(QP), ratio(QP), mont(QP), sfw(QP * 256), sinv(QP * 256),
        rbf((size_t)QP * S2 * N1), rbi((size_t)QP * S2 * N1);
    c.roots.resize(QP);
    for (size_t r = 0; r < QP; ++r) {
        const uint64_t q = moduli[r];
        const uint64_t psi = minimal_root(2 * N, q), ipsi = invmod(psi, q);
        c.roots[r] = psi;
        const uint64_t ni = invmod(N % q, q);
        std::vector<uint64_t> f(N), b(N);
        uint64_t p = 1, ip = 1;
        for (uint32_t i = 0; i < N; ++i) {
            uint32_t k = bitrev(i, (int)c.logN);
            f[k] = p;
            b[k] = ip;
            p = mulmod(p, psi, q);
            ip = mulmod(ip, ipsi, q);
        }
        for (uint32_t i = 0; i < 256 && i < N; ++i) {
            sfw[r * 256 + i] = ntt_pair(f[i], q);
            sinv[r * 256 + i] = ntt_pair(b[i], q);  // before the N^-1 fold below
        }
        for (uint32_t g = 0; g < S2; ++g)
            for (uint32_t k1 = 0; k1 < N1; ++k1) {
                const uint32_t idx = (N1 + k1) << g;  // >= 2: never the folded entry
                rbf[((size_t)r * S2 + g) * N1 + k1] = ntt_pair(f[idx], q);
                rbi[((size_t)r * S2 + g) * N1 + k1] = ntt_pair(b[idx], q);
            }
        b[1] = mulmod(b[1], ni, q);
        for (uint32_t i = 0; i < N; ++i) {
            tw[r * N + i] = ntt_pair(f[i], q);
            itw[r * N + i] = ntt_pair(b[i], q);
        }
        ninv[r] = ntt_pair(ni, q);
        u128 rt = (~(u128)0) / q;  // floor((2^128 - 1) / q) == floor(2^128 / q) for non powers of two
        ratio[r] = ulonglong2{(uint64_t)rt, (uint64_t)(rt >> 64)};
        // Montgomery constants (R = 2^64): -q^-1 mod R (Newton's iteration doubles
        // the correct low bits from the 3 of q^-1 = q mod 8) and R^2 mod q
        uint64_t qi = q;
        for (int it = 0; it < 5; ++it) qi *= 2 - q * qi;
        const u128 r1 = ((~(u128)0) % q + 1) % q;  // 2^128 mod q
        mont[r] = ulonglong2{(uint64_t)0 - qi, (uint64_t)r1};
    }
    c.max_modulus = *std::max_element(c.moduli.begin(), c.moduli.end());
    c.mod = c.upload(c.moduli);
    c.ratio = c.upload(ratio);
    c.mont = c.upload(mont);
    c.tw = c.upload(tw);
    c.itw = c.upload(itw);
    c.ninv = c.upload(ninv);
    c.small_fw = c.upload(sfw);
    c.small_inv = c.upload(sinv);
    c.rb_fw = c.upload(rbf);
    c.rb_inv = c.upload(rbi);
    PFA_HIP(hipDeviceGetAttribute(&c.n_cu, hipDeviceAttributeMultiprocessorCount, c.device));
    PFA_HIP(hipHostMalloc((void **)&c.stage, Ctx::kStageSlots * Ctx::kStageSlotBytes, hipHostMallocDefault));
    for (auto &e : c.stage_ev) PFA_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    // The key-switch inner product splits the items left over after whole
    // rounds of its resident workgroups by digit range; PFA_WS_SLOTS sets the
    // resident count it assumes (tests use it to split small shapes).
    if (const char *w = std::getenv("PFA_WS_SLOTS")) c.ws_slots = (uint32_t)std::max(0, std::atoi(w));
    // Single-launch NTT (N = 2^16, opt-in with PFA_NTT_FLOW=1): built for the
    // round-robin workgroup-to-XCD dealing of a full-chip MI355X partition.
    // PFA_FLOW_WINDOW sets its look-ahead window, PFA_FLOW_WAIT_TICKS its wait
    // bound (tests force an expired wait with it).
    if (const char *w = std::getenv("PFA_FLOW_WINDOW"))
        c.flow_window = (uint32_t)std::min(32, std::max(1, std::atoi(w)));
    if (const char *w = std::getenv("PFA_FLOW_WAIT_TICKS")) c.flow_wait_ticks = (uint32_t)std::max(0, std::atoi(w));
    PFA_HIP(hipHostMalloc((void **)&c.err_host, 64, hipHostMallocMapped));
    *c.err_host = 0;
    PFA_HIP(hipHostGetDevicePointer((void **)&c.err_host_dev, c.err_host, 0));
    c.xcd_rr = xcd_round_robin(c);
    {
        const char *f = std::getenv("PFA_NTT_FLOW");
        const bool want = f ? std::atoi(f) != 0 : false;
        c.ntt_flow = want && c.N == 65536 && c.xcd_rr;
    }

    const uint64_t *Qm = moduli, *Pm = moduli + c.Q;
    const uint32_t alpha = c.P;

    // ModDown constants (src/rns.cu:107-138, src/rns.cu:193-194)
    std::vector<ulonglong2> md_scale_host;
    {
        std::vector<ulonglong2> sc(alpha), pinv(c.Q), pinv_p(c.Q), pq(QP), bc((size_t)alpha * c.Q * 2),
            unit((size_t)c.Q * 2), mdr((size_t)(alpha + 1) * c.Q * 2);
        std::vector<uint64_t> mat((size_t)alpha * c.Q);
        for (uint32_t j = 0; j < alpha; ++j) {
            const uint64_t p = Pm[j];
            sc[j] = ntt_pair(invmod(prod_mod(Pm, alpha, j, p), p), p);
            for (uint32_t i = 0; i < c.Q; ++i) {
                const uint64_t m = prod_mod(Pm, alpha, j, Qm[i]);
                mat[(size_t)j * c.Q + i] = m;
                bc[((size_t)j * c.Q + i) * 2] = ntt_pair(m, Qm[i]);
                bc[((size_t)j * c.Q + i) * 2 + 1] = bconv_pair1(m, Qm[i]);
            }
        }
        for (uint32_t i = 0; i < c.Q; ++i) {
            const uint64_t q = Qm[i];
            const uint64_t pm = prod_mod(Pm, alpha, alpha, q);
            pinv[i] = shoup_pair(invmod(pm, q), q);
            pinv_p[i] = ntt_pair(invmod(pm, q), q);
            pq[i] = shoup_pair(pm, q);
            unit[(size_t)i * 2] = ntt_pair(1 % q, q);
            unit[(size_t)i * 2 + 1] = bconv_pair1(1 % q, q);
            mdr[(size_t)i * 2] = unit[(size_t)i * 2];
            mdr[(size_t)i * 2 + 1] = unit[(size_t)i * 2 + 1];
            for (uint32_t j = 0; j < alpha; ++j) {
                const uint64_t g = invmod(Pm[j] % q, q);
                const size_t k = ((size_t)(1 + j) * c.Q + i) * 2;
                mdr[k] = ntt_pair(g, q);
                mdr[k + 1] = bconv_pair1(g, q);
            }
        }
        for (uint32_t j = 0; j < alpha; ++j) pq[c.Q + j] = ulonglong2{0, 0};
        c.moddown_scale = c.upload(sc);
        c.moddown_mat = c.upload(mat);
        c.pinv = c.upload(pinv);
        c.pmodq = c.upload(pq);
        c.moddown_bc = c.upload(bc);
        c.unit_bc = c.upload(unit);
        c.pinv_p = c.upload(pinv_p);
        c.mdr_bc = c.upload(mdr);
        md_scale_host = sc;
    }

    encoder_init(c);

    // Per-level constants (src/rns.cu:66-95, :141-190)
    c.levels.resize(c.Q + 1);
    for (uint32_t chain = 1; chain <= c.Q; ++chain) {
        Level &lv = c.levels[chain];
        const uint32_t Ql = c.size_Ql(chain), QlP = Ql + alpha;
        lv.Ql = Ql;
        lv.beta = (Ql + alpha - 1) / alpha;
        std::vector<ulonglong2> sc(Ql);
        std::vector<uint64_t> mat((size_t)lv.beta * alpha * QlP, 0);
        std::vector<ulonglong2> bc((size_t)lv.beta * alpha * QlP * 2, ulonglong2{0, 0});
        for (uint32_t b = 0; b < lv.beta; ++b) {
            const uint32_t st = b * alpha, sz = std::min(alpha, Ql - st);
            for (uint32_t i = 0; i < sz; ++i) {
                const uint64_t q = Qm[st + i];
                sc[st + i] = ntt_pair(invmod(prod_mod(Qm + st, sz, i, q), q), q);
                for (uint32_t r = 0; r < QlP; ++r) {
                    const uint64_t p = moduli[c.qlp_row(Ql, r)];
                    const uint64_t m = prod_mod(Qm + st, sz, i, p);
                    const size_t k = ((size_t)b * alpha + i) * QlP + r;
                    mat[k] = m;
                    bc[k * 2] = ntt_pair(m, p);
                    bc[k * 2 + 1] = bconv_pair1(m, p);
                }
            }
        }
        lv.modup_scale = c.upload(sc);
        lv.modup_mat = c.upload(mat);
        lv.modup_bc = c.upload(bc);
        std::vector<ulonglong2> rs(Ql > 1 ? Ql - 1 : 0), rsp(Ql > 1 ? Ql - 1 : 0);
        if (Ql > 1) {
            const uint64_t ql = Qm[Ql - 1];
            for (uint32_t j = 0; j + 1 < Ql; ++j) {
                const uint64_t v = invmod(ql % Qm[j], Qm[j]);
                rs[j] = shoup_pair(v, Qm[j]);
                rsp[j] = ntt_pair(v, Qm[j]);
            }
        }
        lv.rescale_inv = c.upload(rs);
        lv.rescale_inv_p = c.upload(rsp);
        {
            const uint64_t ql = Qm[Ql - 1];
            std::vector<ulonglong2> ms(alpha + 1);
            std::vector<uint64_t> gl(alpha);
            ms[0] = ntt_pair(1 % ql, ql);
            for (uint32_t j = 0; j < alpha; ++j) {
                ms[1 + j] = md_scale_host[j];
                gl[j] = invmod(Pm[j] % ql, ql);
            }
            lv.mdr_scale = c.upload(ms);
            lv.mdr_glast = c.upload(gl);
        }
        {
            std::vector<uint32_t> order, tail;
            for (uint32_t r = 0; r < QlP; ++r)
                (moduli[c.qlp_row(Ql, r)] < kF64PrimeBound ? order : tail).push_back(r);
            order.insert(order.end(), tail.begin(), tail.end());
            lv.ws_order = c.upload(order);
        }
    }
}

// The cached schedule for `key`, built from the item costs `make` returns
// for a grid of R workgroups on first use.
template <class F>
static Sched cached_schedule(const Ctx &c, const std::array<uint32_t, 4> &key, uint32_t R, F make) {
    std::lock_guard<std::mutex> lock(c.sched_mu);
    const auto it = c.scheds.find(key);
    if (it != c.scheds.end()) return it->second;
    const std::vector<uint8_t> cost = make();
    Sched sc;
    const std::vector<uint32_t> perm = lpt_schedule(cost, R);
    if (!perm.empty()) {
        void *p = nullptr;
        PFA_HIP(hipMalloc(&p, perm.size() * sizeof(uint32_t)));
        c.sched_allocs.push_back(p);
        PFA_HIP(hipMemcpy(p, perm.data(), perm.size() * sizeof(uint32_t), hipMemcpyHostToDevice));
        sc = Sched{(const uint32_t *)p, R, (uint32_t)cost.size()};
    }
    c.scheds[key] = sc;
    return sc;
}

// An integer-policy target (a prime of 50 bits or more: Montgomery sums and
// Shoup butterflies) costs about three FP64 ones.
static uint8_t target_cost(const Ctx &c, uint32_t row) { return c.moduli[row] < kF64PrimeBound ? 1 : 3; }

Sched modup_schedule(const Ctx &c, uint32_t chain, uint32_t batch) {
    if (batch == 0 || batch > 64) return {};
    const Level &lv = c.level(chain);
    const uint32_t Ql = lv.Ql, alpha = c.P, QlP = Ql + alpha;
    const uint32_t col_tiles = (1u << (c.logN - c.logN / 2)) / 16u;
    const uint32_t NG = batch * lv.beta * col_tiles, total = grouped_total(NG, QlP);
    const uint32_t R = std::min(total, (uint32_t)c.n_cu * 4u);
    // items (member, digit b's column tile, target position j) in the
    // grouped order of k_bconv_cols; the digit's own limbs are skipped
    return cached_schedule(c, {0u, chain, batch, 0u}, R, [&] {
        std::vector<uint8_t> cost(total, 0);
        for (uint32_t w = 0; w < total; ++w) {
            uint32_t g, j;
            if (!grouped_item(w, NG, QlP, g, j)) continue;
            const uint32_t b = (g / col_tiles) % lv.beta, n_in = std::min(alpha, Ql - b * alpha);
            if (j >= b * alpha && j < b * alpha + n_in) continue;
            cost[w] = target_cost(c, c.qlp_row(Ql, j));
        }
        return cost;
    });
}

Sched epi_schedule(const Ctx &c, uint32_t J, uint32_t M, uint32_t tiles, uint32_t grid) {
    const uint64_t total = (uint64_t)M * J * tiles;
    if (total <= grid || total > (1u << 20) || J > c.Q) return {};
    // item w: row tile w mod tiles of poly (w / tiles) mod M, target (w / tiles) / M
    return cached_schedule(c, {1u, J, M, tiles}, grid, [&] {
        std::vector<uint8_t> cost(total);
        for (uint32_t w = 0; w < total; ++w) cost[w] = target_cost(c, (w / tiles) / M);
        return cost;
    });
}

std::vector<uint32_t> lpt_schedule(const std::vector<uint8_t> &cost, uint32_t R) {
    const uint32_t total = (uint32_t)cost.size();
    if (R == 0 || R % 8 || total <= R) return {};
    std::vector<uint32_t> perm(total, ~0u), used(R, 0), load(R, 0);
    auto npos = [&](uint32_t b) { return (total - b + R - 1) / R; };
    for (uint32_t x = 0; x < 8; ++x) {
        std::vector<uint32_t> items;
        for (uint32_t w = x; w < total; w += 8) items.push_back(w);
        std::stable_sort(items.begin(), items.end(), [&](uint32_t a, uint32_t b) { return cost[a] > cost[b]; });
        // min-heap on (assigned cost, positions, workgroup): ties go to the
        // workgroup with fewer positions, which has fewer items left to take
        using E = std::pair<std::pair<uint32_t, uint32_t>, uint32_t>;
        std::vector<E> heap;
        for (uint32_t b = x; b < R; b += 8)
            if (npos(b)) heap.push_back({{0u, npos(b)}, b});
        auto later = [](const E &a, const E &b) { return a > b; };
        std::make_heap(heap.begin(), heap.end(), later);
        for (uint32_t w : items) {
            if (heap.empty()) return {};
            std::pop_heap(heap.begin(), heap.end(), later);
            const uint32_t b = heap.back().second;
            heap.pop_back();
            perm[b + used[b] * R] = w;
            ++used[b];
            load[b] += cost[w];
            if (used[b] < npos(b)) {
                heap.push_back({{load[b], npos(b)}, b});
                std::push_heap(heap.begin(), heap.end(), later);
            }
        }
    }
    for (uint32_t p : perm)
        if (p == ~0u) return {};
    return perm;
}

Arena &arena_for(const Ctx &c, hipStream_t s) {
    std::lock_guard<std::mutex> lock(c.arena_mu);
    Arena *&a = c.arenas[{std::this_thread::get_id(), s}];
    if (!a) a = new Arena();
    return *a;
}

Scratch::Scratch(const Ctx &c, hipStream_t s) : a_(arena_for(c, s)) {
    marks_.reserve(a_.chunks.size());
    for (auto &ch : a_.chunks) marks_.push_back(ch.top);
}

Scratch::~Scratch() {
    for (size_t i = 0; i < a_.chunks.size(); ++i) a_.chunks[i].top = i < marks_.size() ? marks_[i] : 0;
}

void *Scratch::alloc_bytes(size_t bytes) {
    bytes = (bytes + 255) & ~(size_t)255;
    if (bytes == 0) bytes = 256;
    for (auto &ch : a_.chunks) {
        if (ch.cap - ch.top >= bytes) {
            void *p = ch.base + ch.top;
            ch.top += bytes;
            return p;
        }
    }
    const size_t cap = std::max(bytes, (size_t)256 << 20);
    void *p = nullptr;
    PFA_HIP(hipMalloc(&p, cap));
    a_.chunks.push_back(Arena::Chunk{(char *)p, cap, bytes});
    return p;
}

void upload_async(const Ctx &c, void *dst, const void *src, size_t n, hipStream_t s) {
    if (n == 0) return;
    if (!c.stage || n > Ctx::kStageSlotBytes) {
        PFA_HIP(hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, s));
        return;
    }
    std::lock_guard<std::mutex> lock(c.stage_mu);
    const size_t i = c.stage_next++ % Ctx::kStageSlots;
    PFA_HIP(hipEventSynchronize(c.stage_ev[i]));  // the slot's previous copy is done
    char *slot = c.stage + i * Ctx::kStageSlotBytes;
    std::memcpy(slot, src, n);
    PFA_HIP(hipMemcpyAsync(dst, slot, n, hipMemcpyHostToDevice, s));
    PFA_HIP(hipEventRecord(c.stage_ev[i], s));
}

void upload_parts(const Ctx &c, Scratch &sc, hipStream_t s, std::initializer_list<HostPart> parts, void **dev) {
    size_t total = 0;
    for (const HostPart &p : parts) total += (p.bytes + 15) & ~(size_t)15;
    if (total == 0) return;
    std::vector<char> packed(total);
    char *block = sc.alloc<char>(total);
    size_t off = 0, i = 0;
    for (const HostPart &p : parts) {
        if (p.bytes) std::memcpy(packed.data() + off, p.src, p.bytes);
        dev[i++] = block + off;
        off += (p.bytes + 15) & ~(size_t)15;
    }
    upload_async(c, block, packed.data(), total, s);
}

static void destroy(Ctx *c) {
    if (!c) return;
    int prev = 0;
    (void)hipGetDevice(&prev);
    (void)hipSetDevice(c->device);
    (void)hipDeviceSynchronize();
    for (auto &e : c->stage_ev)
        if (e) (void)hipEventDestroy(e);
    if (c->stage) (void)hipHostFree(c->stage);
    if (c->err_host) (void)hipHostFree(c->err_host);
    for (auto &kv : c->arenas) {
        for (auto &ch : kv.second->chunks) (void)hipFree(ch.base);
        if (kv.second->flow) (void)hipFree(kv.second->flow);
        if (kv.second->ws_counter) (void)hipFree(kv.second->ws_counter);
        delete kv.second;
    }
    for (void *p : c->allocations) (void)hipFree(p);
    for (void *p : c->sched_allocs) (void)hipFree(p);
    (void)hipSetDevice(prev);
    delete c;
}

Ctx *ctx_of(const pfa_context *c) {
    if (!c) fail(PFA_ERR_INVALID_ARGUMENT, "null context");
    check_device_errors(*(const Ctx *)c);
    return (Ctx *)c;
}

void check_device_errors(const Ctx &c) {
    if (!c.err_host) return;
    volatile uint32_t *h = c.err_host;
    const uint32_t bits = *h;
    if (bits == 0) return;
    *h = 0;
    std::string why;
    if (bits & 1u) why += " a single-launch NTT's bounded wait expired;";
    if (bits & 2u) why += " a single-launch NTT ended with tiles not transformed;";
    if (bits & 4u) why += " the digit chunks of one key-switch inner-product item ran on different XCDs;";
    fail(PFA_ERR_RUNTIME, "device error:" + why + " the outputs of the kernels involved and everything computed "
                                                  "from them are invalid");
}

}  // namespace pfa

using namespace pfa;

extern "C" {

const char *pfa_last_error(void) { return g_last_error.c_str(); }

int pfa_abi_version(void) { return 1; }

int pfa_create_coeff_modulus(uint64_t poly_degree, const int *bit_sizes, size_t count, uint64_t *out) {
    return guarded([&] {
        require(bit_sizes && out, "null argument");
        create_coeff_modulus(poly_degree, bit_sizes, count, out);
    });
}

int pfa_context_create(uint64_t poly_degree, const uint64_t *moduli, size_t size_QP, size_t special_size,
                       int device, pfa_context **out) {
    Ctx *c = nullptr;
    int rc = guarded([&] {
        require(moduli && out, "null argument");
        validate(poly_degree, moduli, size_QP, special_size);
        c = new Ctx();
        c->device = device;
        int prev = 0;
        PFA_HIP(hipGetDevice(&prev));
        PFA_HIP(hipSetDevice(device));
        try {
            build(*c, poly_degree, moduli, size_QP, special_size);
            noalloc_init(device);
        } catch (...) {
            (void)hipSetDevice(prev);
            throw;
        }
        PFA_HIP(hipSetDevice(prev));
        *out = (pfa_context *)c;
    });
    if (rc != PFA_OK) destroy(c);
    return rc;
}

void pfa_context_destroy(pfa_context *ctx) { destroy((Ctx *)ctx); }

int pfa_synchronize(const pfa_context *ctx, void *stream) {
    return guarded([&] {
        // checked after the wait only: a record read before it could be
        // followed by more stores of the same still-running kernel
        if (!ctx) fail(PFA_ERR_INVALID_ARGUMENT, "null context");
        const Ctx &c = *(const Ctx *)ctx;
        PFA_HIP(hipStreamSynchronize(as_stream(stream)));
        check_device_errors(c);
    });
}

int pfa_context_roots(const pfa_context *ctx, uint64_t *out) {
    return guarded([&] {
        const Ctx *c = ctx_of(ctx);
        require(out != nullptr, "null argument");
        std::copy(c->roots.begin(), c->roots.end(), out);
    });
}

}  // extern "C"
