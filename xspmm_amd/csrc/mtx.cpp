// mtx.cpp -- MatrixMarket coordinate reader (host).
//
// Same result as the reference's reader, utils/matrix_io.hpp:27-98
// (matrix_utils::io::read_mtx<T>), which the examples use to load real
// matrices (examples/04_real_matrices_benchmark.cpp:104-110):
//   * lines that are empty or whose first character is '%' are skipped;
//   * the first other line gives rows, cols, nnz ("Failed to parse MTX
//     dimensions." otherwise); a file without one is a 0 x 0 matrix;
//   * each later line gives a 1-based row and column; lines where either
//     cannot be read are dropped, and so are entries outside the matrix;
//   * the value is read as a float; when it is absent or unreadable (no
//     digits, a dangling exponent, overflow, inf/nan text) it is 1.0, so
//     pattern files read as ones; symmetric/Hermitian headers are not
//     expanded, complex files keep the real part;
//   * entries are sorted by (row, column); duplicates are kept, in file order;
//   * indices are int, values static_cast<T> of the float.
// The reference extracts each number with std::istringstream; the
// extractors below accept exactly the characters libstdc++ accepts for an
// int and a float and convert with strtof in the C locale, as it does.
// The file is read whole and split into lines once; sorting is a counting
// sort by row followed by a stable sort of each row by column.
#include <hip/hip_fp16.h>
#include <locale.h>

#include <algorithm>
#include <cerrno>
#include <climits>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <numeric>
#include <string>
#include <vector>

#include "internal.hpp"
#include "matrix_io.hpp"

namespace xspmm {
namespace detail {

namespace {

bool is_space(char c)
{
    return c == ' ' || c == '\t' || c == '\n' || c == '\v' || c == '\f' || c == '\r';
}

// `stream >> int`: skip white space, optional sign, decimal digits, the value
// must fit an int.  Returns false (and leaves *v) when no number is read.
bool take_int(const char*& p, const char* end, int* v)
{
    while (p < end && is_space(*p)) ++p;
    const char* q = p;
    bool neg = false;
    if (q < end && (*q == '+' || *q == '-')) neg = *q++ == '-';
    const char* d = q;
    long long x = 0;
    bool big = false;
    while (q < end && *q >= '0' && *q <= '9') {
        x = x * 10 + (*q - '0');
        if (x > (long long)INT_MAX + 1) big = true, x = (long long)INT_MAX + 1;
        ++q;
    }
    if (q == d) return false;
    p = q;
    const long long s = neg ? -x : x;
    if (big || s > INT_MAX || s < INT_MIN) return false;
    *v = (int)s;
    return true;
}

locale_t c_locale()
{
    static locale_t loc = newlocale(LC_ALL_MASK, "C", (locale_t)0);
    return loc;
}

// `stream >> float`: skip white space, then the characters libstdc++ takes
// for a float (sign, digits, one '.', an exponent mark after a digit with an
// optional sign); the token must convert whole to a finite float.
bool take_float(const char*& p, const char* end, float* v)
{
    while (p < end && is_space(*p)) ++p;
    const char* q = p;
    if (q < end && (*q == '+' || *q == '-')) ++q;
    bool mant = false, dot = false, sci = false;
    for (; q < end; ++q) {
        const char c = *q;
        if (c >= '0' && c <= '9') {
            mant = true;
        } else if (c == '.' && !dot && !sci) {
            dot = true;
        } else if ((c == 'e' || c == 'E') && !sci && mant) {
            sci = true;
            if (q + 1 < end && (q[1] == '+' || q[1] == '-')) ++q;
        } else {
            break;
        }
    }
    const size_t n = (size_t)(q - p);
    if (n == 0) return false;
    char buf[128];
    std::string big;
    char* tok = buf;
    if (n >= sizeof(buf)) {
        big.assign(p, n);
        tok = &big[0];
    } else {
        std::memcpy(buf, p, n);
        buf[n] = '\0';
    }
    char* stop = nullptr;
    const float x = strtof_l(tok, &stop, c_locale());
    if (stop != tok + n || std::isinf(x)) return false;
    *v = x;
    return true;
}

}  // namespace

MtxData read_matrix_market(const std::string& path)
{
    std::FILE* f = std::fopen(path.c_str(), "rb");
    if (!f) throw MtxError("Could not open MTX file: " + path);
    std::string text;
    char chunk[1 << 16];
    size_t got;
    while ((got = std::fread(chunk, 1, sizeof(chunk), f)) > 0) text.append(chunk, got);
    std::fclose(f);

    const char* p = text.data();
    const char* const fend = p + text.size();
    auto next_line = [&](const char*& b, const char*& e) -> bool {
        if (p >= fend) return false;
        b = p;
        const void* nl = std::memchr(p, '\n', (size_t)(fend - p));
        e = nl ? static_cast<const char*>(nl) : fend;
        p = nl ? e + 1 : fend;
        return true;
    };

    MtxData m;
    const char *b, *e;
    while (next_line(b, e)) {
        if (b == e || *b == '%') continue;
        int r = 0, c = 0, n = 0;
        const char* q = b;
        if (!(take_int(q, e, &r) && take_int(q, e, &c) && take_int(q, e, &n)))
            throw MtxError("Failed to parse MTX dimensions.");
        m.rows = r;
        m.cols = c;
        if (n > 0) {
            m.r.reserve((size_t)n);
            m.c.reserve((size_t)n);
            m.v.reserve((size_t)n);
        }
        break;
    }
    while (next_line(b, e)) {
        if (b == e || *b == '%') continue;
        const char* q = b;
        int r, c;
        if (!take_int(q, e, &r) || !take_int(q, e, &c)) continue;
        float v = 1.0f;
        if (!take_float(q, e, &v)) v = 1.0f;
        if (r < 1 || r > m.rows || c < 1 || c > m.cols) continue;
        m.r.push_back(r - 1);
        m.c.push_back(c - 1);
        m.v.push_back(v);
    }

    // (row, column) order, equal keys in file order: counting sort by row,
    // then a stable sort of each row by column
    const size_t nnz = m.v.size();
    const int rows = m.rows > 0 ? m.rows : 0;
    m.row_ptr.assign((size_t)rows + 1, 0);
    for (size_t k = 0; k < nnz; ++k) ++m.row_ptr[(size_t)m.r[k] + 1];
    std::partial_sum(m.row_ptr.begin(), m.row_ptr.end(), m.row_ptr.begin());
    std::vector<int> fill(m.row_ptr.begin(), m.row_ptr.end() - 1);
    std::vector<int> idx(nnz);
    for (size_t k = 0; k < nnz; ++k) idx[(size_t)fill[(size_t)m.r[k]]++] = (int)k;
    for (int r = 0; r < rows; ++r) {
        auto first = idx.begin() + m.row_ptr[(size_t)r], last = idx.begin() + m.row_ptr[(size_t)r + 1];
        std::stable_sort(first, last, [&](int a, int b2) { return m.c[(size_t)a] < m.c[(size_t)b2]; });
    }
    m.col_ind.resize(nnz);
    m.values.resize(nnz);
    for (size_t k = 0; k < nnz; ++k) {
        m.col_ind[k] = m.c[(size_t)idx[k]];
        m.values[k] = m.v[(size_t)idx[k]];
    }
    m.r.clear();
    m.r.shrink_to_fit();
    m.c.clear();
    m.c.shrink_to_fit();
    m.v.clear();
    m.v.shrink_to_fit();
    return m;
}

}  // namespace detail
}  // namespace xspmm

namespace matrix_utils {
namespace io {

template <typename T>
HostCSRMatrix<T> read_mtx(const std::string& filename)
{
    auto m = xspmm::detail::read_matrix_market(filename);
    HostCSRMatrix<T> h;
    h.num_rows = m.rows;
    h.num_cols = m.cols;
    h.row_ptr = std::move(m.row_ptr);
    h.col_ind = std::move(m.col_ind);
    h.values.resize(m.values.size());
    for (size_t k = 0; k < m.values.size(); ++k) h.values[k] = static_cast<T>(m.values[k]);
    return h;
}

template HostCSRMatrix<float> read_mtx<float>(const std::string&);
template HostCSRMatrix<double> read_mtx<double>(const std::string&);
template HostCSRMatrix<__half> read_mtx<__half>(const std::string&);

}  // namespace io
}  // namespace matrix_utils
