#pragma once

// MatrixMarket coordinate reader with the interface of the reference's
// utils/matrix_io.hpp:14-98 (namespace matrix_utils::io, HostCSRMatrix<T>,
// read_mtx<T>), implemented in libxspmm.so (instantiated for float, double
// and __half).  The same matrix as the reference's reader: comment and empty
// lines skipped, 1-based entries outside the matrix dropped, missing or
// unreadable values read as 1.0, no symmetric expansion, entries sorted by
// (row, column) with duplicates kept in file order.  Errors are
// std::runtime_error with the reference's messages ("Could not open MTX
// file: <name>", "Failed to parse MTX dimensions.").  The reference header's
// printing helpers are not part of this library.

#include <string>
#include <vector>

namespace matrix_utils {
namespace io {

template <typename T>
struct HostCSRMatrix {
    int num_rows = 0;
    int num_cols = 0;
    std::vector<int> row_ptr;
    std::vector<int> col_ind;
    std::vector<T> values;
};

template <typename T>
HostCSRMatrix<T> read_mtx(const std::string& filename);

}  // namespace io
}  // namespace matrix_utils
