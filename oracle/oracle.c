/*
 * oracle.c -- CPU restatement of the xSpMM SpMM hot path.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h): the product never calls this.
 * Each function cites the reference file:line it restates.  The code is a
 * plain, obviously-sequential restatement; speed matters only for
 * xo_bcsr_spmm_f32, which doubles as the timed CPU baseline.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------ */
/* helpers                                                                  */
/* ------------------------------------------------------------------------ */

/* IEEE binary16 -> binary32, exact for every input (incl. subnormals). */
static inline float h2f(uint16_t h)
{
    uint32_t s = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t f;
    if (e == 0) {
        if (m == 0) {
            f = s;
        } else {
            int sh = 0;
            while (!(m & 0x400u)) { m <<= 1; ++sh; }
            m &= 0x3ffu;
            f = s | ((uint32_t)(113 - sh) << 23) | (m << 13);
        }
    } else if (e == 31) {
        f = s | 0x7f800000u | (m << 13);
    } else {
        f = s | ((e + 112u) << 23) | (m << 13);
    }
    float r;
    memcpy(&r, &f, 4);
    return r;
}

static inline float load_val(const void* base, int64_t i, int vsz)
{
    if (vsz == 2) return h2f(((const uint16_t*)base)[i]);
    return ((const float*)base)[i];
}

static int cmp_i64(const void* a, const void* b)
{
    int64_t x = *(const int64_t*)a, y = *(const int64_t*)b;
    return (x > y) - (x < y);
}

/* ------------------------------------------------------------------------ */
/* CSR -> BCSR   (src/core/conversion.cpp:8-100)                             */
/* ------------------------------------------------------------------------ */

int64_t xo_bcsr_count(int64_t M, int64_t K, int64_t rb, int64_t cb,
                      const int64_t* rp, const int64_t* ci,
                      int64_t* bcsr_row_ptr)
{
    if (rb <= 0 || cb <= 0) return -2;
    int64_t Mb = (M + rb - 1) / rb;          /* conversion.cpp:29 */
    int64_t Kb = (K + cb - 1) / cb;          /* conversion.cpp:30 */
    /* block_map[bc] remembers the last block-row that touched column
     * block bc (conversion.cpp:39, :48-52). */
    int64_t* last = (int64_t*)malloc((size_t)(Kb > 0 ? Kb : 1) * sizeof(int64_t));
    for (int64_t j = 0; j < Kb; ++j) last[j] = -1;
    int64_t total = 0;
    bcsr_row_ptr[0] = 0;
    for (int64_t br = 0; br < Mb; ++br) {
        int64_t r0 = br * rb, r1 = r0 + rb < M ? r0 + rb : M;
        for (int64_t r = r0; r < r1; ++r) {
            for (int64_t idx = rp[r]; idx < rp[r + 1]; ++idx) {
                int64_t c = ci[idx];
                if (c < 0 || c >= K) { free(last); return -1; }
                int64_t bc = c / cb;
                if (last[bc] != br) { last[bc] = br; ++total; }
            }
        }
        bcsr_row_ptr[br + 1] = total;        /* conversion.cpp:66-68 */
    }
    free(last);
    return total;
}

void xo_bcsr_fill(int64_t M, int64_t K, int64_t rb, int64_t cb,
                  const int64_t* rp, const int64_t* ci,
                  const void* vals, int vsz,
                  const int64_t* bcsr_row_ptr,
                  int64_t* bcsr_col_ind, void* bcsr_vals)
{
    int64_t Mb = (M + rb - 1) / rb;
    int64_t Kb = (K + cb - 1) / cb;
    int64_t bsz = rb * cb;
    int64_t* last = (int64_t*)malloc((size_t)(Kb > 0 ? Kb : 1) * sizeof(int64_t));
    int64_t* rank = (int64_t*)malloc((size_t)(Kb > 0 ? Kb : 1) * sizeof(int64_t));
    for (int64_t j = 0; j < Kb; ++j) last[j] = -1;
    unsigned char* out = (unsigned char*)bcsr_vals;
    const unsigned char* in = (const unsigned char*)vals;
    for (int64_t br = 0; br < Mb; ++br) {
        int64_t r0 = br * rb, r1 = r0 + rb < M ? r0 + rb : M;
        int64_t base = bcsr_row_ptr[br];
        int64_t n = 0;
        /* Phase 1: distinct active block columns (conversion.cpp:42-59). */
        for (int64_t r = r0; r < r1; ++r)
            for (int64_t idx = rp[r]; idx < rp[r + 1]; ++idx) {
                int64_t bc = ci[idx] / cb;
                if (last[bc] != br) { last[bc] = br; bcsr_col_ind[base + n++] = bc; }
            }
        /* Sorted ascending (conversion.cpp:61-64). */
        qsort(bcsr_col_ind + base, (size_t)n, sizeof(int64_t), cmp_i64);
        for (int64_t j = 0; j < n; ++j) rank[bcsr_col_ind[base + j]] = j;
        /* Zero-initialised row-major r x c blocks (conversion.cpp:70-73). */
        memset(out + (size_t)(base * bsz) * vsz, 0, (size_t)(n * bsz) * vsz);
        /* Phase 2: scatter in CSR order, so the last duplicate wins
         * (conversion.cpp:75-91, flat index at :84-88). */
        for (int64_t r = r0; r < r1; ++r)
            for (int64_t idx = rp[r]; idx < rp[r + 1]; ++idx) {
                int64_t c = ci[idx];
                int64_t g = base + rank[c / cb];
                int64_t flat = g * bsz + (r % rb) * cb + (c % cb);
                memcpy(out + (size_t)flat * vsz, in + (size_t)idx * vsz, (size_t)vsz);
            }
    }
    free(last);
    free(rank);
}

/* ------------------------------------------------------------------------ */
/* Jaccard clustering   (src/cpu/clustering_sylos_labini.cpp:13-120)        */
/* ------------------------------------------------------------------------ */

/* Distance between a cluster pattern and a row (clustering...cpp:35-46):
 * 1 - |p & q| / |p | q| in float, 0 when the union is empty. */
static float jaccard_dist(const uint64_t* p, const uint64_t* q, int64_t words)
{
    int inter = 0, uni = 0;
    for (int64_t w = 0; w < words; ++w) {
        inter += __builtin_popcountll(p[w] & q[w]);
        uni += __builtin_popcountll(p[w] | q[w]);
    }
    if (uni == 0) return 0.0f;
    return 1.0f - ((float)inter / (float)uni);
}

void xo_jaccard(int64_t M, int64_t K, const int64_t* rp, const int64_t* ci,
                float dist_thresh, int64_t block_width, int64_t* perm)
{
    if (M == 0) return;                                  /* :63 */
    int64_t nblk = (K + block_width - 1) / block_width;  /* :18 */
    int64_t words = (nblk + 63) / 64;                    /* :19 */
    if (words == 0) words = 1;
    uint64_t* q = (uint64_t*)calloc((size_t)(M * words), sizeof(uint64_t));
    /* Quotient rows: bit b of row i set iff row i has a column in block b
     * (:23-31). */
    for (int64_t i = 0; i < M; ++i)
        for (int64_t j = rp[i]; j < rp[i + 1]; ++j) {
            int64_t b = ci[j] / block_width;
            if (ci[j] < 0 || b >= nblk) continue;
            q[i * words + b / 64] |= 1ULL << (b % 64);
        }
    int64_t* un = (int64_t*)malloc((size_t)M * sizeof(int64_t));
    for (int64_t i = 0; i < M; ++i) un[i] = i;           /* :78-82 */
    int64_t n_un = M;
    uint64_t* p = (uint64_t*)malloc((size_t)words * sizeof(uint64_t));
    int64_t out = 0;
    while (n_un > 0) {                                   /* :86 */
        int64_t seed = un[--n_un];                       /* :87-88 */
        perm[out++] = seed;
        memcpy(p, q + seed * words, (size_t)words * sizeof(uint64_t));
        /* Scan from the back; joins swap-remove with the last element
         * (:93-105). */
        for (int64_t i = n_un - 1; i >= 0; --i) {
            int64_t cand = un[i];
            float d = jaccard_dist(p, q + cand * words, words);
            if (d <= dist_thresh) {
                perm[out++] = cand;
                for (int64_t w = 0; w < words; ++w) p[w] |= q[cand * words + w];
                un[i] = un[n_un - 1];
                --n_un;
            }
        }
    }
    /* Clusters are emitted in creation order, members in join order, which
     * is the flattening of :110-116. */
    free(p);
    free(un);
    free(q);
}

/* ------------------------------------------------------------------------ */
/* Row gather / dense scatter                                               */
/* ------------------------------------------------------------------------ */

void xo_apply_perm(int64_t M, const int64_t* rp, const int64_t* ci,
                   const void* vals, int vsz, const int64_t* perm,
                   int64_t* nrp, int64_t* nci, void* nvals)
{
    /* src/cpu/clustering_sylos_labini.cpp:159-171 */
    const unsigned char* in = (const unsigned char*)vals;
    unsigned char* out = (unsigned char*)nvals;
    int64_t pos = 0;
    nrp[0] = 0;
    for (int64_t i = 0; i < M; ++i) {
        int64_t old = perm[i];
        for (int64_t j = rp[old]; j < rp[old + 1]; ++j) {
            nci[pos] = ci[j];
            memcpy(out + (size_t)pos * vsz, in + (size_t)j * vsz, (size_t)vsz);
            ++pos;
        }
        nrp[i + 1] = pos;
    }
}

void xo_unpermute(int64_t M, int64_t N, const float* in, float* out,
                  const int64_t* perm)
{
    /* src/common/permutation.hpp:89-108: out[perm[r]*N + c] = in[r*N + c] */
    for (int64_t r = 0; r < M; ++r)
        memcpy(out + perm[r] * N, in + r * N, (size_t)N * sizeof(float));
}

/* ------------------------------------------------------------------------ */
/* SpMM                                                                     */
/* ------------------------------------------------------------------------ */

void xo_bcsr_spmm_f64(int64_t M, int64_t K, int64_t N, int64_t Mb,
                      const int64_t* brp, const int64_t* bci,
                      const float* bvals, const float* B, double* C)
{
    /* Tile semantics of src/common/spmm_math.hpp:55-127: each 16-row strip of
     * C is overwritten with sum_b A_b * B[16*col_b : +16, :]; strips with no
     * blocks become zero.  Rows >= M are not stored, B rows >= K are absent. */
    memset(C, 0, (size_t)(M * N) * sizeof(double));
    for (int64_t br = 0; br < Mb; ++br)
        for (int64_t b = brp[br]; b < brp[br + 1]; ++b) {
            const float* a = bvals + b * 256;
            for (int64_t i = 0; i < 16; ++i) {
                int64_t row = br * 16 + i;
                if (row >= M) break;
                double* c = C + row * N;
                for (int64_t k = 0; k < 16; ++k) {
                    int64_t kr = bci[b] * 16 + k;
                    if (kr >= K) break;
                    double av = a[i * 16 + k];
                    if (av == 0.0) continue;
                    const float* brow = B + kr * N;
                    for (int64_t n = 0; n < N; ++n) c[n] += av * (double)brow[n];
                }
            }
        }
}

/* AVX2 clone chosen at load time when the host supports it (no FMA, so the
 * rounding is the same as the default clone's). */
__attribute__((target_clones("avx2", "default")))
void xo_bcsr_spmm_f32(int64_t M, int64_t K, int64_t N, int64_t Mb,
                      const int64_t* brp, const int64_t* bci,
                      const void* bvals, const void* B, int vsz, float* C,
                      int nthreads)
{
    /* fp32 B (widened once when the input is fp16). */
    float* Bf = NULL;
    const float* Bp;
    if (vsz == 2) {
        Bf = (float*)malloc((size_t)(K * N) * sizeof(float));
        for (int64_t i = 0; i < K * N; ++i) Bf[i] = h2f(((const uint16_t*)B)[i]);
        Bp = Bf;
    } else {
        Bp = (const float*)B;
    }
#ifdef _OPENMP
    int nt = nthreads > 1 ? nthreads : 1;
#pragma omp parallel for schedule(dynamic, 4) num_threads(nt)
#endif
    for (int64_t br = 0; br < Mb; ++br) {
        float acc[16 * 1024];
        float a[256];
        for (int64_t n0 = 0; n0 < N; n0 += 1024) {
            int64_t nn = N - n0 < 1024 ? N - n0 : 1024;
            memset(acc, 0, sizeof(float) * 16 * (size_t)nn);
            for (int64_t b = brp[br]; b < brp[br + 1]; ++b) {
                for (int e = 0; e < 256; ++e) a[e] = load_val(bvals, b * 256 + e, vsz);
                for (int64_t i = 0; i < 16; ++i) {
                    float* c = acc + i * nn;
                    for (int64_t k = 0; k < 16; ++k) {
                        int64_t kr = bci[b] * 16 + k;
                        if (kr >= K) break;
                        float av = a[i * 16 + k];
                        const float* brow = Bp + kr * N + n0;
                        for (int64_t n = 0; n < nn; ++n) c[n] += av * brow[n];
                    }
                }
            }
            for (int64_t i = 0; i < 16; ++i) {
                int64_t row = br * 16 + i;
                if (row >= M) break;
                memcpy(C + row * N + n0, acc + i * nn, sizeof(float) * (size_t)nn);
            }
        }
    }
    free(Bf);
}

void xo_csr_spmm_f64(int64_t M, int64_t N, const int64_t* rp,
                     const int64_t* ci, const float* vals, const float* B,
                     double* C)
{
    memset(C, 0, (size_t)(M * N) * sizeof(double));
    for (int64_t r = 0; r < M; ++r)
        for (int64_t j = rp[r]; j < rp[r + 1]; ++j) {
            double av = vals[j];
            const float* brow = B + ci[j] * N;
            for (int64_t n = 0; n < N; ++n) C[r * N + n] += av * (double)brow[n];
        }
}

void xo_errors(int64_t n, const float* actual, const double* expected,
               double* out)
{
    /* utils/matrix_compare.hpp:29-64 (computed in fp64 here). */
    double max_abs = 0, max_rel = 0, ssd = 0, sse = 0;
    for (int64_t i = 0; i < n; ++i) {
        double e = expected[i], a = actual[i];
        double d = a - e, ad = fabs(d);
        if (ad > max_abs) max_abs = ad;
        double rel = fabs(e) > 0 ? ad / fabs(e) : ad;
        if (rel > max_rel) max_rel = rel;
        ssd += d * d;
        sse += e * e;
    }
    double fe = sqrt(ssd), fr = sqrt(sse);
    out[0] = max_abs;
    out[1] = max_rel;
    out[2] = fe;
    out[3] = fr > 0 ? fe / fr : fe;
}

int xo_max_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
