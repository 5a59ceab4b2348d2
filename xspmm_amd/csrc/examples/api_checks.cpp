// api_checks.cpp -- exercises the C++ drop-in API the way the reference's
// examples do (examples/01_uspmm_checkers.cpp, 05_core_spmm_benchmark.cpp,
// 06_bad_col_lengths.cpp), with host closed forms / host products as the
// expected values instead of rocSPARSE / rocBLAS.  Prints one PASS/FAIL line
// per check and exits non-zero if any check fails.
#include <hip/hip_fp16.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <memory>
#include <numeric>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

#include <xspmm/clustering.hpp>
#include <xspmm/core/executor.hpp>
#include <xspmm/matrix/conversion.hpp>
#include <xspmm/plan.hpp>
#include <xspmm/xspmm.hpp>

namespace {

int failures = 0;

void report(const std::string& name, bool ok, const std::string& detail = "")
{
    std::printf("[%s] %s %s\n", ok ? "PASS" : "FAIL", name.c_str(), detail.c_str());
    std::fflush(stdout);
    if (!ok) ++failures;
}

std::string sci(double v)
{
    char b[32];
    std::snprintf(b, sizeof(b), "%.2e", v);
    return b;
}

template <typename I>
struct HostCsr {
    I M = 0, K = 0;
    std::vector<I> rp, ci;
    std::vector<float> vals;
};

// utils/matrix_gen.hpp:185-211 shape (checkers), rows shuffled.
template <typename I>
HostCsr<I> checkers(I M, I K, I bs, unsigned seed)
{
    std::mt19937 rng(seed);
    std::uniform_real_distribution<float> u(0.1f, 1.0f);
    std::vector<std::vector<I>> rows((size_t)M);
    for (I i = 0; i < M; ++i)
        for (I j = 0; j < K; ++j)
            if ((i / bs + j / bs) % 2 == 1) rows[(size_t)i].push_back(j);
    std::vector<I> order((size_t)M);
    std::iota(order.begin(), order.end(), I(0));
    std::shuffle(order.begin(), order.end(), rng);
    HostCsr<I> h;
    h.M = M;
    h.K = K;
    h.rp.push_back(0);
    for (I r : order) {
        for (I c : rows[(size_t)r]) {
            h.ci.push_back(c);
            h.vals.push_back(u(rng));
        }
        h.rp.push_back((I)h.ci.size());
    }
    return h;
}

// utils/matrix_gen.hpp:69-90 shape (banded).
template <typename I>
HostCsr<I> banded(I M, I bw, unsigned seed)
{
    std::mt19937 rng(seed);
    std::uniform_real_distribution<float> u(0.1f, 1.0f);
    HostCsr<I> h;
    h.M = h.K = M;
    h.rp.push_back(0);
    for (I i = 0; i < M; ++i) {
        for (I j = std::max<I>(0, i - bw); j <= std::min<I>(M - 1, i + bw); ++j) {
            h.ci.push_back(j);
            h.vals.push_back(u(rng));
        }
        h.rp.push_back((I)h.ci.size());
    }
    return h;
}

// The banded shape with one extra column per row, far from the band: every
// block-row then has a gap, so Tier-1 keeps the column-batch kernel.
template <typename I>
HostCsr<I> banded_gap(I M, I bw, unsigned seed)
{
    std::mt19937 rng(seed);
    std::uniform_real_distribution<float> u(0.1f, 1.0f);
    HostCsr<I> h;
    h.M = h.K = M;
    h.rp.push_back(0);
    for (I i = 0; i < M; ++i) {
        const I lo = std::max<I>(0, i - bw), hi = std::min<I>(M - 1, i + bw);
        const I far = (I)((i + M / 2) % M);
        if (far < lo) {
            h.ci.push_back(far);
            h.vals.push_back(u(rng));
        }
        for (I j = lo; j <= hi; ++j) {
            h.ci.push_back(j);
            h.vals.push_back(u(rng));
        }
        if (far > hi) {
            h.ci.push_back(far);
            h.vals.push_back(u(rng));
        }
        h.rp.push_back((I)h.ci.size());
    }
    return h;
}

template <typename I>
std::vector<double> row_sums(const HostCsr<I>& h)
{
    std::vector<double> s((size_t)h.M, 0.0);
    for (I r = 0; r < h.M; ++r)
        for (I k = h.rp[(size_t)r]; k < h.rp[(size_t)r + 1]; ++k) s[(size_t)r] += h.vals[(size_t)k];
    return s;
}

double rel_frob_vs_rowsums(const std::vector<float>& C, const std::vector<double>& rs, size_t N)
{
    double num = 0, den = 0;
    for (size_t r = 0; r < rs.size(); ++r)
        for (size_t j = 0; j < N; ++j) {
            const double d = C[r * N + j] - rs[r];
            num += d * d;
            den += rs[r] * rs[r];
        }
    return std::sqrt(num) / std::max(std::sqrt(den), 1e-300);
}

template <typename T>
std::vector<T> convert_vals(const std::vector<float>& v)
{
    std::vector<T> out(v.size());
    for (size_t i = 0; i < v.size(); ++i) out[i] = T(v[i]);
    return out;
}

template <typename T, typename I>
xspmm::CSRMatrix<T, I> upload(std::shared_ptr<const xspmm::Executor> ex, const HostCsr<I>& h,
                              std::vector<T>& vals_out)
{
    vals_out = convert_vals<T>(h.vals);
    xspmm::CSRMatrix<T, I> A(ex, h.M, h.K, (I)h.ci.size());
    A.copy_from_host(h.rp.data(), h.ci.data(), vals_out.data());
    return A;
}

// examples/01: cluster + permute + convert + Tier-1 + host unpermute.
template <typename T, typename I>
void check_checkers_manual(std::shared_ptr<const xspmm::Executor> ex, const char* tname)
{
    const I M = 1024, K = 1024, N = 256;
    auto h = checkers<I>(M, K, 4, 42);
    std::vector<T> hv;
    auto A = upload<T, I>(ex, h, hv);
    I* d_perm = nullptr;
    ex->allocate(reinterpret_cast<void**>(&d_perm), sizeof(I) * (size_t)M);
    xspmm::compute_1d_jaccard_clustering(ex, A, 0.5f, (I)16, d_perm);
    auto A_opt = xspmm::apply_permutation(ex, A, d_perm);
    auto A_b = xspmm::csr_to_bcsr(ex, A_opt, (I)16, (I)16);
    std::vector<T> hB((size_t)K * N, T(1.0f));
    T* d_B = nullptr;
    float* d_C = nullptr;
    ex->allocate(reinterpret_cast<void**>(&d_B), sizeof(T) * hB.size());
    ex->allocate(reinterpret_cast<void**>(&d_C), sizeof(float) * (size_t)M * N);
    ex->copy_from_host(d_B, hB.data(), sizeof(T) * hB.size());
    xspmm::spmm(A_b, d_B, d_C, N);
    ex->synchronize();
    std::vector<float> Cp((size_t)M * N), C((size_t)M * N);
    std::vector<I> perm((size_t)M);
    ex->copy_to_host(Cp.data(), d_C, sizeof(float) * Cp.size());
    ex->copy_to_host(perm.data(), d_perm, sizeof(I) * perm.size());
    for (I i = 0; i < M; ++i)
        std::copy(Cp.begin() + (size_t)i * N, Cp.begin() + (size_t)(i + 1) * N,
                  C.begin() + (size_t)perm[(size_t)i] * N);
    const auto rs = row_sums(h);
    double max_abs = 0;
    for (I r = 0; r < M; ++r)
        for (I j = 0; j < N; ++j) max_abs = std::max(max_abs, std::abs(C[(size_t)r * N + j] - rs[(size_t)r]));
    const double rf = rel_frob_vs_rowsums(C, rs, N);
    const double tol = sizeof(T) == 2 ? 2e-3 : 1e-5;
    // fp16 values are rounded before the sum; the row sums use the fp32 values
    report(std::string("checkers manual pipeline ") + tname,
           rf < tol && (sizeof(T) == 2 || max_abs < 1e-3),
           "rel_frob=" + std::to_string(rf) + " max_abs=" + std::to_string(max_abs));
    ex->free(d_perm);
    ex->free(d_B);
    ex->free(d_C);
}

// Tier-2 automated pipeline with timings.
template <typename T, typename I>
void check_tier2(std::shared_ptr<const xspmm::Executor> ex, bool cluster, const char* tname)
{
    const I M = 1024, N = 64;
    auto h = checkers<I>(M, M, 4, 7);
    std::vector<T> hv;
    auto A = upload<T, I>(ex, h, hv);
    std::vector<T> hB((size_t)M * N, T(1.0f));
    T* d_B = nullptr;
    float* d_C = nullptr;
    ex->allocate(reinterpret_cast<void**>(&d_B), sizeof(T) * hB.size());
    ex->allocate(reinterpret_cast<void**>(&d_C), sizeof(float) * (size_t)M * N);
    ex->copy_from_host(d_B, hB.data(), sizeof(T) * hB.size());
    xspmm::SpMMTimings t;
    t.clustering_ms = -1.0;  // untouched when clustering is off
    xspmm::spmm(ex, A, d_B, d_C, N, (I)16, cluster, &t);
    std::vector<float> C((size_t)M * N);
    ex->copy_to_host(C.data(), d_C, sizeof(float) * C.size());
    std::vector<double> rs((size_t)M, 0.0);
    for (I r = 0; r < M; ++r)
        for (I k = h.rp[(size_t)r]; k < h.rp[(size_t)r + 1]; ++k) rs[(size_t)r] += (float)hv[(size_t)k];
    const double rf = rel_frob_vs_rowsums(C, rs, N);
    const bool timing_ok = t.total_pipeline_ms > 0 && t.spmm_ms > 0 &&
                           (cluster ? t.clustering_ms > 0 : t.clustering_ms == -1.0);
    report(std::string("tier2 pipeline ") + (cluster ? "clustered " : "plain ") + tname,
           rf < 1e-5 && timing_ok,
           "rel_frob=" + std::to_string(rf) + " total_ms=" + std::to_string(t.total_pipeline_ms));
    ex->free(d_B);
    ex->free(d_C);
}

// examples/06: ragged N on a banded matrix, B = ones.
template <typename T, typename I>
void check_ragged_n(std::shared_ptr<const xspmm::Executor> ex, const char* tname)
{
    const I M = 2048;
    auto h = banded<I>(M, 40, 3);
    std::vector<T> hv;
    auto A = upload<T, I>(ex, h, hv);
    auto Ab = xspmm::csr_to_bcsr(ex, A, (I)16, (I)16);
    std::vector<double> rs((size_t)M, 0.0);
    for (I r = 0; r < M; ++r)
        for (I k = h.rp[(size_t)r]; k < h.rp[(size_t)r + 1]; ++k) rs[(size_t)r] += (float)hv[(size_t)k];
    bool ok = true;
    std::string worst;
    for (I N : {1, 2, 4, 8, 17, 18, 24, 30, 31, 128}) {
        std::vector<T> hB((size_t)M * N, T(1.0f));
        T* d_B = nullptr;
        float* d_C = nullptr;
        ex->allocate(reinterpret_cast<void**>(&d_B), sizeof(T) * hB.size());
        ex->allocate(reinterpret_cast<void**>(&d_C), sizeof(float) * (size_t)M * N);
        ex->copy_from_host(d_B, hB.data(), sizeof(T) * hB.size());
        xspmm::spmm(Ab, d_B, d_C, N);
        ex->synchronize();
        std::vector<float> C((size_t)M * N);
        ex->copy_to_host(C.data(), d_C, sizeof(float) * C.size());
        const double rf = rel_frob_vs_rowsums(C, rs, (size_t)N);
        if (!(rf < 1e-5)) {
            ok = false;
            worst += " N=" + std::to_string(N) + ":" + std::to_string(rf);
        }
        ex->free(d_B);
        ex->free(d_C);
    }
    report(std::string("ragged N banded ") + tname, ok, worst);
}

// A grid of more than 2048 block-rows: csr_to_bcsr computes the fp16 Tier-1
// dispatch order once (the matrix owns it, a move hands it over); Tier-1 C
// with it equals C from the same blocks without it (copy_from_host drops the
// order, so that call orders the rows itself), and the row sums.
template <typename I>
void check_dispatch_order(std::shared_ptr<const xspmm::Executor> ex, const char* tname)
{
    const I M = 40000, N = 64;
    auto h = banded_gap<I>(M, 20, 5);
    std::vector<__half> hv;
    auto A = upload<__half, I>(ex, h, hv);
    auto Ab = xspmm::csr_to_bcsr(ex, A, (I)16, (I)16);
    bool ok = Ab.get_dispatch_order() != nullptr && !Ab.get_band_rows();
    auto Am = std::move(Ab);
    ok = ok && Am.get_dispatch_order() != nullptr && Ab.get_dispatch_order() == nullptr;
    const I Mb = Am.get_num_block_rows(), nnzb = Am.get_num_blocks();
    std::vector<I> brp((size_t)Mb + 1), bci((size_t)nnzb);
    std::vector<__half> bv((size_t)nnzb * 256);
    ex->copy_to_host(brp.data(), Am.get_bcsr_row_ptr(), sizeof(I) * brp.size());
    ex->copy_to_host(bci.data(), Am.get_bcsr_col_ind(), sizeof(I) * bci.size());
    ex->copy_to_host(bv.data(), Am.get_bcsr_values(), sizeof(__half) * bv.size());
    xspmm::BCSRMatrix<__half, I> Ac(ex, Mb, Am.get_num_block_cols(), nnzb, 16, 16);
    Ac.set_shape(M, M);
    Ac.copy_from_host(brp.data(), bci.data(), bv.data());
    ok = ok && Ac.get_dispatch_order() == nullptr;
    std::vector<__half> hB((size_t)M * N, __half(1.0f));
    __half* d_B = nullptr;
    float *d_C1 = nullptr, *d_C2 = nullptr;
    ex->allocate(reinterpret_cast<void**>(&d_B), sizeof(__half) * hB.size());
    ex->allocate(reinterpret_cast<void**>(&d_C1), sizeof(float) * (size_t)M * N);
    ex->allocate(reinterpret_cast<void**>(&d_C2), sizeof(float) * (size_t)M * N);
    ex->copy_from_host(d_B, hB.data(), sizeof(__half) * hB.size());
    xspmm::spmm(Am, d_B, d_C1, N);
    xspmm::spmm(Ac, d_B, d_C2, N);
    ex->synchronize();
    std::vector<float> C1((size_t)M * N), C2((size_t)M * N);
    ex->copy_to_host(C1.data(), d_C1, sizeof(float) * C1.size());
    ex->copy_to_host(C2.data(), d_C2, sizeof(float) * C2.size());
    ex->free(d_B);
    ex->free(d_C1);
    ex->free(d_C2);
    ok = ok && std::memcmp(C1.data(), C2.data(), sizeof(float) * C1.size()) == 0;
    std::vector<double> rs((size_t)M, 0.0);
    for (I r = 0; r < M; ++r)
        for (I k = h.rp[(size_t)r]; k < h.rp[(size_t)r + 1]; ++k) rs[(size_t)r] += (float)hv[(size_t)k];
    const double rf = rel_frob_vs_rowsums(C1, rs, (size_t)N);
    report(std::string("cached dispatch order ") + tname, ok && rf < 1e-5,
           "rel_frob " + std::to_string(rf));
}

// examples/05 shape (fp16 and fp32): csr_to_bcsr finds the contiguous block-rows and
// keeps the band flag on the matrix (moved with it, cleared by
// copy_from_host); Tier-1 then runs the band kernel.  A hand-filled copy with
// the flag set gives the same C bit for bit, without it the column-batch
// kernel's C (fp32 summation order apart).
template <typename T, typename I>
void check_band_rows(std::shared_ptr<const xspmm::Executor> ex, const char* tname)
{
    const I M = 4096, N = 128;
    auto h = banded<I>(M, 300, 9);
    std::vector<T> hv;
    auto A = upload<T, I>(ex, h, hv);
    auto Ab = xspmm::csr_to_bcsr(ex, A, (I)16, (I)16);
    bool ok = Ab.get_band_rows();
    auto Am = std::move(Ab);
    ok = ok && Am.get_band_rows();
    const I Mb = Am.get_num_block_rows(), nnzb = Am.get_num_blocks();
    std::vector<I> brp((size_t)Mb + 1), bci((size_t)nnzb);
    std::vector<T> bv((size_t)nnzb * 256);
    ex->copy_to_host(brp.data(), Am.get_bcsr_row_ptr(), sizeof(I) * brp.size());
    ex->copy_to_host(bci.data(), Am.get_bcsr_col_ind(), sizeof(I) * bci.size());
    ex->copy_to_host(bv.data(), Am.get_bcsr_values(), sizeof(T) * bv.size());
    xspmm::BCSRMatrix<T, I> Ac(ex, Mb, Am.get_num_block_cols(), nnzb, 16, 16);
    Ac.set_shape(M, M);
    Ac.set_band_rows(true);
    Ac.copy_from_host(brp.data(), bci.data(), bv.data());
    ok = ok && !Ac.get_band_rows();  // copy_from_host clears it
    std::vector<T> hB((size_t)M * N, T(1.0f));
    T* d_B = nullptr;
    float *d_C1 = nullptr, *d_C2 = nullptr, *d_C3 = nullptr;
    ex->allocate(reinterpret_cast<void**>(&d_B), sizeof(T) * hB.size());
    ex->allocate(reinterpret_cast<void**>(&d_C1), sizeof(float) * (size_t)M * N);
    ex->allocate(reinterpret_cast<void**>(&d_C2), sizeof(float) * (size_t)M * N);
    ex->allocate(reinterpret_cast<void**>(&d_C3), sizeof(float) * (size_t)M * N);
    ex->copy_from_host(d_B, hB.data(), sizeof(T) * hB.size());
    xspmm::spmm(Am, d_B, d_C1, N);  // band kernel
    xspmm::spmm(Ac, d_B, d_C2, N);  // column-batch kernel
    Ac.set_band_rows(true);         // the rows are contiguous: the caller may say so
    xspmm::spmm(Ac, d_B, d_C3, N);  // band kernel
    ex->synchronize();
    std::vector<float> C1((size_t)M * N), C2((size_t)M * N), C3((size_t)M * N);
    ex->copy_to_host(C1.data(), d_C1, sizeof(float) * C1.size());
    ex->copy_to_host(C2.data(), d_C2, sizeof(float) * C2.size());
    ex->copy_to_host(C3.data(), d_C3, sizeof(float) * C3.size());
    ex->free(d_B);
    ex->free(d_C1);
    ex->free(d_C2);
    ex->free(d_C3);
    ok = ok && std::memcmp(C1.data(), C3.data(), sizeof(float) * C1.size()) == 0;
    std::vector<double> rs((size_t)M, 0.0);
    for (I r = 0; r < M; ++r)
        for (I k = h.rp[(size_t)r]; k < h.rp[(size_t)r + 1]; ++k) rs[(size_t)r] += (float)hv[(size_t)k];
    const double rf1 = rel_frob_vs_rowsums(C1, rs, (size_t)N);
    const double rf2 = rel_frob_vs_rowsums(C2, rs, (size_t)N);
    report(std::string("band kernel from csr_to_bcsr ") + tname, ok && rf1 < 1e-5 && rf2 < 1e-5,
           "rel_frob band " + sci(rf1) + ", column batches " + sci(rf2));
}

// CPU and GPU conversions of the same matrix agree bit for bit.
template <typename I>
void check_cpu_gpu_conversion(std::shared_ptr<const xspmm::Executor> gpu)
{
    auto cpu = std::make_shared<xspmm::CpuExecutor>();
    auto h = checkers<I>(300, 257, 3, 11);
    std::vector<float> hv;
    auto Ac = upload<float, I>(cpu, h, hv);
    auto Ag = upload<float, I>(gpu, h, hv);
    auto Bc = xspmm::csr_to_bcsr(cpu, Ac, (I)16, (I)16);
    auto Bg = xspmm::csr_to_bcsr(gpu, Ag, (I)16, (I)16);
    auto Bgc = xspmm::csr_to_bcsr(cpu, Ag, (I)16, (I)16);  // GPU input, CPU target
    bool ok = Bc.get_num_blocks() == Bg.get_num_blocks() && Bc.get_num_blocks() == Bgc.get_num_blocks();
    if (ok) {
        const size_t nb = (size_t)Bc.get_num_blocks(), Mb = (size_t)Bc.get_num_block_rows();
        std::vector<I> rp((Mb + 1)), ci(nb);
        std::vector<float> v(nb * 256);
        gpu->copy_to_host(rp.data(), Bg.get_bcsr_row_ptr(), sizeof(I) * (Mb + 1));
        gpu->copy_to_host(ci.data(), Bg.get_bcsr_col_ind(), sizeof(I) * nb);
        gpu->copy_to_host(v.data(), Bg.get_bcsr_values(), sizeof(float) * v.size());
        ok = std::equal(rp.begin(), rp.end(), Bc.get_bcsr_row_ptr()) &&
             std::equal(ci.begin(), ci.end(), Bc.get_bcsr_col_ind()) &&
             std::memcmp(v.data(), Bc.get_bcsr_values(), sizeof(float) * v.size()) == 0 &&
             std::memcmp(Bgc.get_bcsr_values(), Bc.get_bcsr_values(), sizeof(float) * v.size()) == 0 &&
             Bg.get_num_rows() == 300 && Bg.get_num_cols() == 257;
    }
    report("cpu/gpu conversion bit-exact", ok);
}

void check_errors(std::shared_ptr<const xspmm::Executor> gpu)
{
    auto cpu = std::make_shared<xspmm::CpuExecutor>();
    bool ok1 = false, ok2 = false, ok3 = false, ok4 = false;
    try {
        xspmm::CSRMatrix<float, int> bad(cpu, -1, 4, 0);
    } catch (const std::invalid_argument&) {
        ok1 = true;
    }
    try {
        xspmm::BCSRMatrix<float, int> b(cpu, 2, 2, 1, 16, 16);
        xspmm::spmm(b, (const float*)nullptr, (float*)nullptr, 16);
    } catch (const std::runtime_error& e) {
        ok2 = std::string(e.what()).find("CPU SpMM fallback is not yet implemented") != std::string::npos;
    }
    try {
        xspmm::CudaExecutor c(0);
    } catch (const std::runtime_error&) {
        ok3 = true;
    }
    try {
        xspmm::BCSRMatrix<float, int> b(gpu, 1, 1, 0, 8, 8);
        xspmm::spmm(b, (const float*)nullptr, (float*)nullptr, 16);
    } catch (const std::invalid_argument&) {
        ok4 = true;
    }
    report("error behaviour", ok1 && ok2 && ok3 && ok4,
           std::to_string(ok1) + std::to_string(ok2) + std::to_string(ok3) + std::to_string(ok4));
}

// Prepared product: a plan's C equals the pipeline's C bit for bit, for
// several N, after the source matrix is gone and after a move.
template <typename T, typename I>
void check_plan(std::shared_ptr<const xspmm::Executor> ex, bool cluster, const char* tname)
{
    const I M = 1000, N = 72;
    auto h = checkers<I>(M, M, 4, 11);
    std::vector<T> hv;
    std::vector<T> hB((size_t)M * N);
    std::mt19937 rng(3);
    std::uniform_real_distribution<float> u(-1.0f, 1.0f);
    for (auto& b : hB) b = T(u(rng));
    T* d_B = nullptr;
    float *d_C1 = nullptr, *d_C2 = nullptr;
    ex->allocate(reinterpret_cast<void**>(&d_B), sizeof(T) * hB.size());
    ex->allocate(reinterpret_cast<void**>(&d_C1), sizeof(float) * (size_t)M * N);
    ex->allocate(reinterpret_cast<void**>(&d_C2), sizeof(float) * (size_t)M * N);
    ex->copy_from_host(d_B, hB.data(), sizeof(T) * hB.size());
    bool ok = true;
    std::string detail;
    xspmm::SpMMTimings t;
    std::unique_ptr<xspmm::SpMMPlan<T, I>> plan;
    {
        auto A = upload<T, I>(ex, h, hv);
        plan = std::make_unique<xspmm::SpMMPlan<T, I>>(ex, A, (I)16, cluster, &t);
    }  // A freed: the plan keeps its own copies
    xspmm::SpMMPlan<T, I> moved(std::move(*plan));
    for (I n : {N, (I)8, (I)13, N}) {
        std::vector<float> c1((size_t)M * n), c2((size_t)M * n);
        {
            auto A2 = upload<T, I>(ex, h, hv);
            xspmm::spmm(ex, A2, d_B, d_C1, n, (I)16, cluster, nullptr);
        }
        moved.execute(d_B, d_C2, n);
        ex->synchronize();
        ex->copy_to_host(c1.data(), d_C1, sizeof(float) * c1.size());
        ex->copy_to_host(c2.data(), d_C2, sizeof(float) * c2.size());
        if (std::memcmp(c1.data(), c2.data(), sizeof(float) * c1.size()) != 0) {
            ok = false;
            detail += " mismatch at N=" + std::to_string((long long)n);
        }
    }
    ok = ok && moved.get_num_blocks() > 0 && moved.is_clustered() == cluster &&
         (moved.get_permutation() != nullptr) == cluster && t.total_pipeline_ms > 0 &&
         (!cluster || t.clustering_ms > 0);
    report(std::string("prepared plan ") + (cluster ? "clustered " : "plain ") + tname, ok,
           detail + " prep_ms=" + std::to_string(t.total_pipeline_ms));
    ex->free(d_B);
    ex->free(d_C1);
    ex->free(d_C2);
}

}  // namespace

int main()
{
    try {
        auto ex = std::make_shared<xspmm::HipExecutor>(0);
        check_checkers_manual<float, int32_t>(ex, "f32/i32");
        check_checkers_manual<__half, int64_t>(ex, "f16/i64");
        check_tier2<float, int32_t>(ex, true, "f32/i32");
        check_tier2<float, int64_t>(ex, false, "f32/i64");
        check_tier2<__half, int32_t>(ex, true, "f16/i32");
        check_tier2<__half, int64_t>(ex, false, "f16/i64");
        check_ragged_n<float, int32_t>(ex, "f32/i32");
        check_ragged_n<__half, int32_t>(ex, "f16/i32");
        check_dispatch_order<int32_t>(ex, "i32");
        check_dispatch_order<int64_t>(ex, "i64");
        check_band_rows<__half, int32_t>(ex, "f16/i32");
        check_band_rows<__half, int64_t>(ex, "f16/i64");
        check_band_rows<float, int32_t>(ex, "f32/i32");
        check_cpu_gpu_conversion<int32_t>(ex);
        check_cpu_gpu_conversion<int64_t>(ex);
        check_errors(ex);
        check_plan<__half, int32_t>(ex, true, "f16/i32");
        check_plan<__half, int64_t>(ex, false, "f16/i64");
        check_plan<float, int32_t>(ex, true, "f32/i32");
    } catch (const std::exception& e) {
        std::printf("[FAIL] exception: %s\n", e.what());
        return 2;
    }
    std::printf("%s: %d failure(s)\n", failures ? "FAILED" : "OK", failures);
    return failures ? 1 : 0;
}
