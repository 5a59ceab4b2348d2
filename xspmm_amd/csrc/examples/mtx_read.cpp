// mtx_read.cpp -- reads one MatrixMarket file through the C++ interface of
// the reference's utils/matrix_io.hpp (matrix_utils::io::read_mtx<float>) and
// prints "rows cols nnz sum(row_ptr) sum(col_ind) sum(values)", or the error
// message with exit status 1.  Host only: no GPU work.
#include <cstdio>
#include <exception>

#include <matrix_io.hpp>

int main(int argc, char** argv)
{
    if (argc != 2) {
        std::printf("usage: mtx_read FILE\n");
        return 2;
    }
    try {
        auto h = matrix_utils::io::read_mtx<float>(argv[1]);
        long long rs = 0, cs = 0;
        double vs = 0.0;
        for (int x : h.row_ptr) rs += x;
        for (int x : h.col_ind) cs += x;
        for (float v : h.values) vs += (double)v;
        std::printf("%d %d %zu %lld %lld %.17g\n", h.num_rows, h.num_cols, h.values.size(), rs, cs,
                    vs);
        return 0;
    } catch (const std::exception& e) {
        std::printf("%s\n", e.what());
        return 1;
    }
}
