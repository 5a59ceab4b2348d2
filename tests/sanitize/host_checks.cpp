// host_checks.cpp -- the library's host-only code under AddressSanitizer and
// UndefinedBehaviorSanitizer (built and run by tests/test_host_sanitizers.py).
//
//   * the host Jaccard clustering (xspmm_amd/csrc/cluster.cpp), both engines
//     and the automatic choice, 1 and 4 threads, against the C oracle's
//     restatement of the reference greedy (oracle/oracle.c xo_jaccard): the
//     permutations must be equal;
//   * the C oracle's conversion, permutation, un-permutation and products on
//     random inputs (memory safety; their values are checked by
//     tests/test_oracle.py);
//   * the MatrixMarket reader (xspmm_amd/csrc/mtx.cpp) on every file named on
//     the command line, as float, double and __half (errors are caught and
//     printed: malformed files must raise, not read out of bounds).
// Prints "host checks ok" and exits 0 when every comparison holds.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <exception>
#include <string>
#include <vector>

#include <hip/hip_fp16.h>

#include "matrix_io.hpp"
#include "oracle.h"

namespace xspmm {
namespace detail {
template <typename I>
void jaccard_clustering_host(int64_t M, int64_t K, const I* rp, const I* ci, float dist_thresh,
                             int64_t block_width, I* perm, int nthreads);
}
}  // namespace xspmm

namespace {

struct Rng {
    uint64_t s;
    uint64_t next()
    {
        s ^= s << 13;
        s ^= s >> 7;
        s ^= s << 17;
        return s;
    }
    int64_t below(int64_t n) { return n > 0 ? (int64_t)(next() % (uint64_t)n) : 0; }
};

struct Csr {
    int64_t M = 0, K = 0;
    std::vector<int64_t> rp, ci;
    std::vector<float> vals;
};

// rows of Binomial-like length, some empty, unsorted columns and duplicates
Csr random_csr(Rng& r, int64_t M, int64_t K, int64_t max_len)
{
    Csr c;
    c.M = M;
    c.K = K;
    c.rp.push_back(0);
    for (int64_t i = 0; i < M; ++i) {
        const int64_t len = K > 0 && r.below(5) ? r.below(max_len + 1) : 0;
        for (int64_t e = 0; e < len; ++e) {
            c.ci.push_back(r.below(K));
            c.vals.push_back((float)(r.below(7) - 3));
        }
        c.rp.push_back((int64_t)c.ci.size());
    }
    return c;
}

int failures = 0;

void check(bool ok, const std::string& what)
{
    if (!ok) {
        ++failures;
        std::printf("FAILED: %s\n", what.c_str());
    }
}

void clustering_cases()
{
    Rng r{0x9e3779b97f4a7c15ull};
    const int64_t shapes[][3] = {{1, 1, 1},    {17, 40, 6},   {300, 500, 12},
                                 {1000, 3000, 30}, {257, 64, 64}, {64, 1, 1}};
    const float thresholds[] = {0.0f, 0.3f, 0.5f, 0.9f, 1.0f};
    const int64_t widths[] = {1, 16, 64};
    const char* engines[] = {"scan", "index", "auto"};
    int cases = 0;
    for (const auto& sh : shapes)
        for (float t : thresholds)
            for (int64_t bw : widths) {
                const Csr c = random_csr(r, sh[0], sh[1], sh[2]);
                std::vector<int64_t> want((size_t)c.M);
                xo_jaccard(c.M, c.K, c.rp.data(), c.ci.data(), t, bw, want.data());
                std::vector<int32_t> rp32(c.rp.begin(), c.rp.end()), ci32(c.ci.begin(), c.ci.end());
                for (const char* eng : engines)
                    for (int nt : {1, 4}) {
                        setenv("XSPMM_CLUSTER_ENGINE", eng, 1);
                        std::vector<int64_t> got((size_t)c.M, -1);
                        xspmm::detail::jaccard_clustering_host<int64_t>(
                            c.M, c.K, c.rp.data(), c.ci.data(), t, bw, got.data(), nt);
                        std::vector<int32_t> got32((size_t)c.M, -1);
                        xspmm::detail::jaccard_clustering_host<int32_t>(
                            c.M, c.K, rp32.data(), ci32.data(), t, bw, got32.data(), nt);
                        bool same = got == want;
                        for (size_t i = 0; i < got32.size(); ++i) same &= got32[i] == want[i];
                        check(same, "clustering M=" + std::to_string(c.M) + " K=" +
                                        std::to_string(c.K) + " t=" + std::to_string(t) +
                                        " bw=" + std::to_string(bw) + " engine=" + eng +
                                        " threads=" + std::to_string(nt));
                        ++cases;
                    }
            }
    unsetenv("XSPMM_CLUSTER_ENGINE");
    std::printf("clustering: %d cases\n", cases);
}

void oracle_cases()
{
    Rng r{12345};
    int cases = 0;
    for (int64_t M : {1, 16, 17, 100}) {
        for (int64_t K : {1, 16, 33, 200}) {
            const Csr c = random_csr(r, M, K, 9);
            const int64_t Mb = (M + 15) / 16;
            std::vector<int64_t> brp((size_t)Mb + 1);
            const int64_t nnzb = xo_bcsr_count(M, K, 16, 16, c.rp.data(), c.ci.data(), brp.data());
            check(nnzb >= 0, "bcsr count");
            std::vector<int64_t> bci((size_t)(nnzb > 0 ? nnzb : 1));
            std::vector<float> bv((size_t)(nnzb > 0 ? nnzb : 1) * 256);
            xo_bcsr_fill(M, K, 16, 16, c.rp.data(), c.ci.data(), c.vals.data(), 4, brp.data(),
                         bci.data(), bv.data());
            for (int64_t N : {1, 7, 64}) {
                std::vector<float> B((size_t)(K * N));
                for (auto& x : B) x = (float)(r.below(5) - 2);
                std::vector<double> C64((size_t)(M * N)), Ccsr((size_t)(M * N));
                std::vector<float> C32((size_t)(M * N));
                xo_bcsr_spmm_f64(M, K, N, Mb, brp.data(), bci.data(), bv.data(), B.data(), C64.data());
                xo_bcsr_spmm_f32(M, K, N, Mb, brp.data(), bci.data(), bv.data(), B.data(), 4,
                                 C32.data(), 2);
                // duplicates: the BCSR keeps the last one, the CSR product sums
                // them, so the two only agree on the shape checks here
                xo_csr_spmm_f64(M, N, c.rp.data(), c.ci.data(), c.vals.data(), B.data(), Ccsr.data());
                double err[4];
                xo_errors(M * N, C32.data(), C64.data(), err);
                check(err[0] == 0.0, "f32 and f64 products of small integers agree");
                std::vector<int64_t> perm((size_t)M);
                xo_jaccard(M, K, c.rp.data(), c.ci.data(), 0.5f, 16, perm.data());
                std::vector<int64_t> nrp((size_t)M + 1), nci(c.ci.size() + 1);
                std::vector<float> nv(c.vals.size() + 1);
                xo_apply_perm(M, c.rp.data(), c.ci.data(), c.vals.data(), 4, perm.data(), nrp.data(),
                              nci.data(), nv.data());
                check(nrp[(size_t)M] == c.rp[(size_t)M], "permutation keeps nnz");
                std::vector<float> U((size_t)(M * N));
                xo_unpermute(M, N, C32.data(), U.data(), perm.data());
                ++cases;
            }
        }
    }
    // a column outside [0, K): count reports it
    std::vector<int64_t> rp = {0, 2}, ci = {0, 5}, brp(2);
    check(xo_bcsr_count(1, 5, 16, 16, rp.data(), ci.data(), brp.data()) == -1, "bad column");
    std::printf("oracle: %d cases\n", cases);
}

template <typename T>
void read_one(const char* path, const char* type)
{
    try {
        const auto m = matrix_utils::io::read_mtx<T>(path);
        // negative dimensions read as an empty matrix (no rows, no entries)
        const size_t rows = m.num_rows > 0 ? (size_t)m.num_rows : 0;
        check(m.row_ptr.size() == rows + 1, std::string("row_ptr size ") + path);
        check(m.row_ptr.back() == (int)m.values.size(), std::string("row_ptr end ") + path);
        check(m.col_ind.size() == m.values.size(), std::string("entries ") + path);
        std::printf("mtx %s (%s): %d x %d, %zu entries\n", path, type, m.num_rows, m.num_cols,
                    m.values.size());
    } catch (const std::exception& e) {
        std::printf("mtx %s (%s): error: %s\n", path, type, e.what());
    }
}

}  // namespace

int main(int argc, char** argv)
{
    clustering_cases();
    oracle_cases();
    for (int i = 1; i < argc; ++i) {
        read_one<float>(argv[i], "float");
        read_one<double>(argv[i], "double");
        read_one<__half>(argv[i], "half");
    }
    if (failures) {
        std::printf("%d failures\n", failures);
        return 1;
    }
    std::printf("host checks ok\n");
    return 0;
}
