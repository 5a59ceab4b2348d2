// cluster.cpp -- host 1-D Jaccard ("Sylos Labini") row clustering.
//
// Exact restatement of the reference greedy (src/cpu/clustering_sylos_labini.cpp:51-120):
//   q_i = bitmap of the block_width-wide column blocks row i touches (:13-33);
//   unclustered = [0..M-1]; while non-empty: seed = pop_back(); p = q_seed;
//   for i = size-1 down to 0: cand = unclustered[i];
//     d = |p|q| == 0 ? 0 : 1 - (float)|p&q| / (float)|p|q|          (:35-46)
//     if d <= dist_thresh: join cand, p |= q_cand,
//                          unclustered[i] = back(), pop_back()       (:97-104)
//   perm = clusters in creation order, members in join order (:110-116).
//
// The visiting order of a seed's scan is "positions of `unclustered` as they
// were when the seed was popped, descending": a swap-remove at position i only
// moves an element that was already visited into slot i.  Both engines below
// reproduce that order and the float comparison exactly, so the permutation
// equals the reference's bit for bit.
//
//  * scan:  the reference loop with the candidate tests of a stretch of
//           positions evaluated in parallel against the current pattern; the
//           joiners down to the first one that grows the pattern are
//           committed (those above it lie inside the pattern and leave it
//           unchanged) and the scan resumes below it.  A popcount bound (d >= 1 - min(|p|,|q|)/max(|p|,|q|), which is
//           monotone under float rounding) skips most bitmap work.
//  * index: for 0 <= dist_thresh < 1 a row can only join a cluster whose
//           pattern shares a block with it (d = 1 otherwise), or an empty
//           pattern if it is empty itself.  Candidates come from per-block row
//           lists; |p&q| is counted through the lists, |p|q| = |p|+|q|-|p&q|.
//           Work is sum over blocks of list length^2 instead of M^2 * words.
// `auto` picks the engine with the smaller estimated cost; the environment
// variable XSPMM_CLUSTER_ENGINE=scan|index forces one (used by the tests).
#include <algorithm>
#include <atomic>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <immintrin.h>
#include <queue>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "internal.hpp"

namespace xspmm {
namespace detail {

namespace {

inline float jaccard_distance(int64_t inter, int64_t uni)
{
    if (uni == 0) return 0.0f;
    return 1.0f - (static_cast<float>(inter) / static_cast<float>(uni));
}

// The test jaccard_distance(inter, uni) <= t, decided without the division
// away from the threshold.  With x = inter / uni (exact), the float value
// RN(1 - RN(x)) is within 2^-23 of 1 - x, so it is <= t whenever
// x >= 1 - t + 2^-23 and > t whenever x < 1 - t - 2^-23; the factors a_hi /
// a_lo add 2^-20 on either side, which also covers the rounding of a * uni.
// That needs inter and uni exact in float (below 2^24); larger counts, and
// the band between the factors, take the division as the reference does.
struct JaccardTest {
    float t, a_hi, a_lo;
    explicit JaccardTest(float thr) : t(thr), a_hi((1.0f - thr) + 0x1p-20f), a_lo((1.0f - thr) - 0x1p-20f) {}
    bool close(int64_t inter, int64_t uni) const
    {
        if (uni == 0) return 0.0f <= t;
        if (uni < (int64_t(1) << 24)) {
            const float fi = static_cast<float>(inter), fu = static_cast<float>(uni);
            if (fi >= a_hi * fu) return true;
            if (fi < a_lo * fu) return false;
        }
        return jaccard_distance(inter, uni) <= t;
    }
    // false when no rows with popcounts mn <= mx can be close (x <= mn / mx)
    bool may_close(int64_t mn, int64_t mx) const
    {
        if (mx >= (int64_t(1) << 24)) return jaccard_distance(mn, mx) <= t;
        return !(static_cast<float>(mn) < a_lo * static_cast<float>(mx));
    }
};

// One thread's share of the scan engine's search: the highest position in
// [bot, top] whose row is close to the pattern p (popcount pc), or -1.
// |p | q| = |p| + |q| - |p & q|, so only the intersection is counted.  The
// AVX-512 instance (vpopcntq, 8 words per instruction) runs when the host CPU
// has the VPOPCNTDQ extension; both instances return the same position.
struct ScanArgs {
    const uint64_t* bits;   // row bitmaps, W words each
    const int32_t* count;   // their popcounts
    const int64_t* un;      // position -> row
    const uint64_t* p;      // pattern
    int64_t W, pc;
};

inline int64_t and_popcount(const uint64_t* a, const uint64_t* b, int64_t n)
{
    int64_t s = 0;
    for (int64_t w = 0; w < n; ++w) s += __builtin_popcountll(a[w] & b[w]);
    return s;
}

__attribute__((target("avx512f,avx512vpopcntdq"))) inline int64_t and_popcount_avx512(
    const uint64_t* a, const uint64_t* b, int64_t n)
{
    __m512i acc = _mm512_setzero_si512();
    int64_t w = 0;
    for (; w + 8 <= n; w += 8)
        acc = _mm512_add_epi64(acc, _mm512_popcnt_epi64(_mm512_and_si512(
                                        _mm512_loadu_si512(a + w), _mm512_loadu_si512(b + w))));
    int64_t s = _mm512_reduce_add_epi64(acc);
    for (; w < n; ++w) s += __builtin_popcountll(a[w] & b[w]);
    return s;
}

// Joiners whose row lies inside the pattern (|p & q| = |q|) leave it as it
// is, so the search goes on past them: it returns the highest position whose
// row joins and grows the pattern, and appends the positions above it whose
// rows join inside the pattern to `inside` (in visiting order).
template <bool AVX512, typename JT>
inline int64_t scan_down(const ScanArgs& a, const JT& jt, int64_t top, int64_t bot,
                         std::vector<int64_t>& inside)
{
    for (int64_t pos = top; pos >= bot; --pos) {
        const int64_t cand = a.un[pos];
        const int64_t qc = a.count[cand];
        const int64_t mn = qc < a.pc ? qc : a.pc, mx = qc < a.pc ? a.pc : qc;
        if (!jt.may_close(mn, mx)) continue;  // cannot reach t
        const uint64_t* q = a.bits + cand * a.W;
        int64_t inter;
        if constexpr (AVX512)
            inter = and_popcount_avx512(a.p, q, a.W);
        else
            inter = and_popcount(a.p, q, a.W);
        if (jt.close(inter, a.pc + qc - inter)) {
            if (inter != qc) return pos;
            inside.push_back(pos);
        }
    }
    return -1;
}

struct Patterns {
    int64_t M = 0, nblk = 0, words = 0;
    std::vector<uint64_t> bits;   // M * words
    std::vector<int32_t> count;   // popcount per row
    const uint64_t* row(int64_t i) const { return bits.data() + i * words; }
};

template <typename I>
Patterns build_patterns(int64_t M, int64_t K, const I* rp, const I* ci, int64_t bw)
{
    Patterns P;
    P.M = M;
    P.nblk = (K + bw - 1) / bw;
    P.words = (P.nblk + 63) / 64;
    if (P.words == 0) P.words = 1;
    P.bits.assign((size_t)(M * P.words), 0ULL);
    P.count.assign((size_t)M, 0);
    for (int64_t i = 0; i < M; ++i) {
        uint64_t* q = P.bits.data() + i * P.words;
        for (int64_t j = (int64_t)rp[i]; j < (int64_t)rp[i + 1]; ++j) {
            const int64_t c = (int64_t)ci[j];
            if (c < 0 || c >= K) throw std::invalid_argument("clustering: column index out of range.");
            const int64_t b = c / bw;
            q[b >> 6] |= 1ULL << (b & 63);
        }
        int32_t n = 0;
        for (int64_t w = 0; w < P.words; ++w) n += __builtin_popcountll(q[w]);
        P.count[(size_t)i] = n;
    }
    return P;
}

// Minimal fork-join pool: run(f) calls f(t) for t in [0, n) on n threads
// (t = 0 on the caller) and returns when all are done.
class Pool {
public:
    explicit Pool(int n) : n_(n < 1 ? 1 : n) {
        for (int t = 1; t < n_; ++t) th_.emplace_back([this, t] { worker(t); });
    }
    ~Pool() {
        stop_.store(true, std::memory_order_release);
        gen_.fetch_add(1, std::memory_order_acq_rel);
        for (auto& t : th_) t.join();
    }
    int size() const { return n_; }
    void run(const std::function<void(int)>& f) {
        if (n_ == 1) {
            f(0);
            return;
        }
        task_ = &f;
        pending_.store(n_ - 1, std::memory_order_release);
        gen_.fetch_add(1, std::memory_order_acq_rel);
        f(0);
        while (pending_.load(std::memory_order_acquire) != 0) std::this_thread::yield();
    }

private:
    void worker(int t) {
        uint64_t seen = 0;
        for (;;) {
            uint64_t g;
            int spins = 0;
            while ((g = gen_.load(std::memory_order_acquire)) == seen) {
                if (++spins > 64) std::this_thread::yield();
            }
            seen = g;
            if (stop_.load(std::memory_order_acquire)) return;
            (*task_)(t);
            pending_.fetch_sub(1, std::memory_order_acq_rel);
        }
    }
    int n_;
    std::vector<std::thread> th_;
    std::atomic<uint64_t> gen_{0};
    std::atomic<int> pending_{0};
    std::atomic<bool> stop_{false};
    const std::function<void(int)>* task_ = nullptr;
};

template <typename JT>
int64_t scan_down_scalar(const ScanArgs& a, const JT& jt, int64_t top, int64_t bot,
                         std::vector<int64_t>& inside)
{
    return scan_down<false>(a, jt, top, bot, inside);
}

template <typename JT>
__attribute__((target("avx512f,avx512vpopcntdq"))) int64_t scan_down_avx512(
    const ScanArgs& a, const JT& jt, int64_t top, int64_t bot, std::vector<int64_t>& inside)
{
    return scan_down<true>(a, jt, top, bot, inside);
}

// XSPMM_CLUSTER_SIMD=scalar forces the scalar search (for tests and CPUs
// where the extension is reported but unwanted).
bool host_has_vpopcntdq()
{
    if (const char* e = std::getenv("XSPMM_CLUSTER_SIMD"))
        if (std::strcmp(e, "scalar") == 0) return false;
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512vpopcntdq");
}

template <typename I>
void engine_scan(const Patterns& P, float t, I* perm, int nthreads)
{
    const int64_t M = P.M, W = P.words;
    const JaccardTest jt(t);
    const bool avx512 = host_has_vpopcntdq();
    std::vector<int64_t> un((size_t)M);
    for (int64_t i = 0; i < M; ++i) un[(size_t)i] = i;
    int64_t n_un = M, out = 0;
    std::vector<uint64_t> p((size_t)W);
    Pool pool(nthreads);
    const int nt = pool.size();
    std::vector<int64_t> found((size_t)nt);
    std::vector<std::vector<int64_t>> inside((size_t)nt);
    // positions searched per round before the range doubles: about 1024 per
    // thread, so that a round's work outweighs waking the pool
    const int64_t first_stretch = std::max<int64_t>(2048, 1024 * (int64_t)nt);

    while (n_un > 0) {
        const int64_t seed = un[(size_t)--n_un];
        perm[out++] = (I)seed;
        std::memcpy(p.data(), P.row(seed), (size_t)W * sizeof(uint64_t));
        int64_t pc = P.count[(size_t)seed];
        int64_t hi = n_un - 1;  // next position to visit
        int64_t stretch = first_stretch;
        while (hi >= 0) {
            // First joining position in [lo, hi] that grows the pattern,
            // scanning downwards, and the joiners inside the pattern above it.
            const int64_t lo = hi - stretch + 1 > 0 ? hi - stretch + 1 : 0;
            const ScanArgs sa{P.bits.data(), P.count.data(), un.data(), p.data(), W, pc};
            auto scan = [&](int64_t top, int64_t bot, std::vector<int64_t>& in) {
                return avx512 ? scan_down_avx512(sa, jt, top, bot, in)
                              : scan_down_scalar(sa, jt, top, bot, in);
            };
            int64_t hit = -1;
            const int64_t len = hi - lo + 1;
            int used = 1;  // shares whose inside-joiners are kept, from the top
            for (auto& v : inside) v.clear();
            if (nt == 1 || len < 4 * nt) {
                hit = scan(hi, lo, inside[0]);
            } else {
                pool.run([&](int tid) {
                    const int64_t per = (len + nt - 1) / nt;
                    const int64_t top = hi - (int64_t)tid * per;
                    const int64_t bot = top - per + 1 > lo ? top - per + 1 : lo;
                    found[(size_t)tid] = top >= bot ? scan(top, bot, inside[(size_t)tid]) : -1;
                });
                // the shares run from the top down: the first share that
                // found a growing joiner ends the stretch
                used = nt;
                for (int k = 0; k < nt; ++k)
                    if (found[(size_t)k] >= 0) {
                        hit = found[(size_t)k];
                        used = k + 1;
                        break;
                    }
            }
            // Joiners inside the pattern above `hit` (or in the whole stretch),
            // in visiting order, with the reference's swap-removes: each moves
            // a row from above (already visited) into the freed position.
            for (int k = 0; k < used; ++k)
                for (const int64_t pos : inside[(size_t)k]) {
                    perm[out++] = (I)un[(size_t)pos];
                    un[(size_t)pos] = un[(size_t)(n_un - 1)];
                    --n_un;
                }
            if (hit < 0) {
                hi = lo - 1;
                stretch *= 2;
                continue;
            }
            const int64_t cand = un[(size_t)hit];
            perm[out++] = (I)cand;
            const uint64_t* q = P.row(cand);
            pc = 0;
            for (int64_t w = 0; w < W; ++w) {
                p[(size_t)w] |= q[w];
                pc += __builtin_popcountll(p[(size_t)w]);
            }
            un[(size_t)hit] = un[(size_t)(n_un - 1)];
            --n_un;
            hi = hit - 1;
            stretch = first_stretch;
        }
    }
}

template <typename I>
void engine_index(const Patterns& P, float t, I* perm, int nthreads)
{
    // Requires 0 <= t < 1 (checked by the caller).
    const int64_t M = P.M, W = P.words, NB = P.nblk;
    const JaccardTest jt(t);
    // Row lists per block (CSR of the transposed pattern).
    std::vector<int64_t> start((size_t)NB + 1, 0);
    for (int64_t i = 0; i < M; ++i) {
        const uint64_t* q = P.row(i);
        for (int64_t w = 0; w < W; ++w)
            for (uint64_t b = q[w]; b; b &= b - 1) ++start[(size_t)(w * 64 + __builtin_ctzll(b)) + 1];
    }
    for (int64_t b = 0; b < NB; ++b) start[(size_t)b + 1] += start[(size_t)b];
    std::vector<int64_t> rows((size_t)start[(size_t)NB]);
    {
        std::vector<int64_t> fill(start.begin(), start.end() - 1);
        for (int64_t i = 0; i < M; ++i) {
            const uint64_t* q = P.row(i);
            for (int64_t w = 0; w < W; ++w)
                for (uint64_t b = q[w]; b; b &= b - 1)
                    rows[(size_t)fill[(size_t)(w * 64 + __builtin_ctzll(b))]++] = i;
        }
    }

    // Partner lists, all rows in parallel: row j is a partner of row i
    // (j != i) when d(q_i, q_j) <= t.  Until its first join a cluster's
    // pattern is q_seed, so a seed none of whose partners is still
    // unclustered stays alone, and the greedy skips its search.  pn[i] = -1:
    // the list was not kept (more than kPartnerCap partners, or an empty row).
    constexpr int kPartnerCap = 32;
    std::vector<int32_t> pn((size_t)M, -1);
    std::vector<int64_t> plist((size_t)M * kPartnerCap);
    {
        Pool pool(nthreads);
        const int nt = pool.size();
        pool.run([&](int tid) {
            std::vector<int32_t> c((size_t)M, 0);
            std::vector<int64_t> seen;
            for (int64_t i = tid; i < M; i += nt) {
                const int64_t ci = P.count[(size_t)i];
                if (ci == 0) continue;
                const uint64_t* q = P.row(i);
                for (int64_t w = 0; w < W; ++w)
                    for (uint64_t b = q[w]; b; b &= b - 1) {
                        const int64_t blk = w * 64 + __builtin_ctzll(b);
                        for (int64_t k = start[(size_t)blk]; k < start[(size_t)blk + 1]; ++k) {
                            const int64_t r = rows[(size_t)k];
                            if (r != i && c[(size_t)r]++ == 0) seen.push_back(r);
                        }
                    }
                int32_t np = 0;
                for (const int64_t r : seen) {
                    const int64_t inter = c[(size_t)r];
                    c[(size_t)r] = 0;
                    if (!jt.close(inter, ci + P.count[(size_t)r] - inter)) continue;
                    if (np < kPartnerCap) plist[(size_t)i * kPartnerCap + np] = r;
                    ++np;
                }
                seen.clear();
                pn[(size_t)i] = np > kPartnerCap ? -1 : np;
            }
        });
    }

    std::vector<int64_t> un((size_t)M), pos((size_t)M);
    for (int64_t i = 0; i < M; ++i) un[(size_t)i] = pos[(size_t)i] = i;
    std::vector<uint8_t> done((size_t)M, 0);
    std::vector<int32_t> cnt((size_t)M, 0);  // |p & q_row| for touched rows
    std::vector<int64_t> touched;
    std::vector<uint64_t> p((size_t)W);
    int64_t n_un = M, out = 0;

    auto remove_at = [&](int64_t at) {  // swap-remove, as the reference does
        const int64_t moved = un[(size_t)(n_un - 1)];
        un[(size_t)at] = moved;
        pos[(size_t)moved] = at;
        --n_un;
    };

    while (n_un > 0) {
        const int64_t seed = un[(size_t)(n_un - 1)];
        --n_un;
        done[(size_t)seed] = 1;
        perm[out++] = (I)seed;
        if (P.count[(size_t)seed] == 0) {
            // Empty pattern: exactly the remaining empty rows join, in
            // descending position order; the pattern stays empty.
            std::vector<std::pair<int64_t, int64_t>> empties;
            for (int64_t k = 0; k < n_un; ++k) {
                const int64_t r = un[(size_t)k];
                if (P.count[(size_t)r] == 0) empties.emplace_back(k, r);
            }
            std::sort(empties.begin(), empties.end(),
                      [](const auto& a, const auto& b) { return a.first > b.first; });
            for (const auto& e : empties) {
                perm[out++] = (I)e.second;
                done[(size_t)e.second] = 1;
                remove_at(pos[(size_t)e.second]);
            }
            continue;
        }
        if (pn[(size_t)seed] >= 0) {
            bool any = false;
            for (int32_t k = 0; k < pn[(size_t)seed] && !any; ++k)
                any = !done[(size_t)plist[(size_t)seed * kPartnerCap + k]];
            if (!any) continue;  // no unclustered partner: a cluster of one
        }
        std::memcpy(p.data(), P.row(seed), (size_t)W * sizeof(uint64_t));
        int64_t pc = P.count[(size_t)seed];
        std::priority_queue<std::pair<int64_t, int64_t>> heap;  // (position, row), max first
        int64_t limit = n_un;  // only positions below `limit` are unvisited
        auto touch_block = [&](int64_t b) {
            for (int64_t k = start[(size_t)b]; k < start[(size_t)b + 1]; ++k) {
                const int64_t r = rows[(size_t)k];
                if (done[(size_t)r]) continue;
                if (cnt[(size_t)r]++ == 0) {
                    touched.push_back(r);
                    if (pos[(size_t)r] < limit) heap.emplace(pos[(size_t)r], r);
                }
            }
        };
        for (int64_t w = 0; w < W; ++w)
            for (uint64_t b = p[(size_t)w]; b; b &= b - 1) touch_block(w * 64 + __builtin_ctzll(b));
        while (!heap.empty()) {
            const auto top = heap.top();
            heap.pop();
            const int64_t at = top.first, r = top.second;
            limit = at;
            const int64_t inter = cnt[(size_t)r];
            const int64_t uni = pc + P.count[(size_t)r] - inter;
            if (!jt.close(inter, uni)) continue;
            perm[out++] = (I)r;
            done[(size_t)r] = 1;
            remove_at(at);
            const uint64_t* q = P.row(r);
            for (int64_t w = 0; w < W; ++w) {
                uint64_t add = q[w] & ~p[(size_t)w];
                p[(size_t)w] |= q[w];
                for (; add; add &= add - 1) {
                    ++pc;
                    touch_block(w * 64 + __builtin_ctzll(add));
                }
            }
        }
        for (int64_t r : touched) cnt[(size_t)r] = 0;
        touched.clear();
    }
}

}  // namespace

template <typename I>
void jaccard_clustering_host(int64_t M, int64_t K, const I* rp, const I* ci, float dist_thresh,
                             int64_t block_width, I* perm, int nthreads)
{
    if (M < 0 || K < 0) throw std::invalid_argument("CSR dimensions must be non-negative.");
    if (M == 0) return;  // reference :63
    if (block_width <= 0) throw std::invalid_argument("clustering: block_width must be positive.");
    if (nthreads <= 0) {
        const unsigned hc = std::thread::hardware_concurrency();
        nthreads = hc ? (int)(hc < 32 ? hc : 32) : 1;
    }
    const Patterns P = build_patterns(M, K, rp, ci, block_width);

    std::string engine = "auto";
    if (const char* e = std::getenv("XSPMM_CLUSTER_ENGINE")) engine = e;
    const bool index_ok = dist_thresh >= 0.0f && dist_thresh < 1.0f;
    if (engine == "auto") {
        // Estimated work: scan ~ M^2/2 * words * 2 / threads word ops;
        // index ~ 3 * sum over blocks of (rows touching the block)^2.
        double scan_cost = 0.5 * (double)M * (double)M * (double)P.words * 2.0 / nthreads;
        std::vector<int64_t> per_block((size_t)P.nblk, 0);
        for (int64_t i = 0; i < M; ++i) {
            const uint64_t* q = P.row(i);
            for (int64_t w = 0; w < P.words; ++w)
                for (uint64_t b = q[w]; b; b &= b - 1) ++per_block[(size_t)(w * 64 + __builtin_ctzll(b))];
        }
        double index_cost = 0;
        for (int64_t v : per_block) index_cost += 3.0 * (double)v * (double)v;
        engine = (index_ok && index_cost < scan_cost) ? "index" : "scan";
    }
    if (engine == "index" && index_ok)
        engine_index<I>(P, dist_thresh, perm, nthreads);
    else
        engine_scan<I>(P, dist_thresh, perm, nthreads);
}

template void jaccard_clustering_host<int32_t>(int64_t, int64_t, const int32_t*, const int32_t*,
                                               float, int64_t, int32_t*, int);
template void jaccard_clustering_host<int64_t>(int64_t, int64_t, const int64_t*, const int64_t*,
                                               float, int64_t, int64_t*, int);

}  // namespace detail
}  // namespace xspmm
