#pragma once
// Device-resident BCSR matrix: bcsr_row_ptr[Mb+1], bcsr_col_ind[nnzb] (block
// columns, ascending within a block-row) and bcsr_values[nnzb*r*c] (each block
// row-major).  Interface as in the reference (include/xspmm/matrix/bcsr.hpp:12-116).
//
// Added to the reference interface: the element shape (get_num_rows /
// get_num_cols).  csr_to_bcsr records the CSR's M and K, so SpMM masks the
// rows and columns of ragged edge blocks instead of touching memory outside
// B and C.  A matrix built directly from the constructor reports the padded
// shape Mb*r x Kb*c, which is what the reference's kernel assumes.

#include <cstdint>
#include <memory>
#include <stdexcept>
#include <utility>

#include "xspmm/core/executor.hpp"

namespace xspmm {

template <typename ValueType, typename IndexType = int64_t>
class BCSRMatrix {
public:
    BCSRMatrix(std::shared_ptr<const Executor> exec, IndexType num_block_rows,
               IndexType num_block_cols, IndexType num_blocks, IndexType r_block, IndexType c_block)
        : exec_(std::move(exec)),
          num_block_rows_(num_block_rows), num_block_cols_(num_block_cols), num_blocks_(num_blocks),
          r_block_(r_block), c_block_(c_block),
          num_rows_(num_block_rows * r_block), num_cols_(num_block_cols * c_block)
    {
        if (num_block_rows < 0 || num_block_cols < 0 || num_blocks < 0) {
            throw std::invalid_argument("BCSR dimensions must be non-negative.");
        }
        exec_->allocate(reinterpret_cast<void**>(&bcsr_row_ptr_),
                        (static_cast<size_t>(num_block_rows) + 1) * sizeof(IndexType));
        if (num_blocks > 0) {
            exec_->allocate(reinterpret_cast<void**>(&bcsr_col_ind_),
                            static_cast<size_t>(num_blocks) * sizeof(IndexType));
            exec_->allocate(reinterpret_cast<void**>(&bcsr_values_), value_bytes());
        }
    }

    ~BCSRMatrix() { release(); }

    BCSRMatrix(const BCSRMatrix&) = delete;
    BCSRMatrix& operator=(const BCSRMatrix&) = delete;

    BCSRMatrix(BCSRMatrix&& o) noexcept
        : exec_(std::move(o.exec_)),
          num_block_rows_(o.num_block_rows_), num_block_cols_(o.num_block_cols_), num_blocks_(o.num_blocks_),
          r_block_(o.r_block_), c_block_(o.c_block_), num_rows_(o.num_rows_), num_cols_(o.num_cols_),
          bcsr_row_ptr_(o.bcsr_row_ptr_), bcsr_col_ind_(o.bcsr_col_ind_), bcsr_values_(o.bcsr_values_),
          dispatch_order_(o.dispatch_order_), band_rows_(o.band_rows_)
    {
        o.bcsr_row_ptr_ = nullptr;
        o.bcsr_col_ind_ = nullptr;
        o.bcsr_values_ = nullptr;
        o.dispatch_order_ = nullptr;
    }

    BCSRMatrix& operator=(BCSRMatrix&& o) noexcept {
        if (this != &o) {
            release();
            exec_ = std::move(o.exec_);
            num_block_rows_ = o.num_block_rows_;
            num_block_cols_ = o.num_block_cols_;
            num_blocks_ = o.num_blocks_;
            r_block_ = o.r_block_;
            c_block_ = o.c_block_;
            num_rows_ = o.num_rows_;
            num_cols_ = o.num_cols_;
            bcsr_row_ptr_ = o.bcsr_row_ptr_;
            bcsr_col_ind_ = o.bcsr_col_ind_;
            bcsr_values_ = o.bcsr_values_;
            dispatch_order_ = o.dispatch_order_;
            band_rows_ = o.band_rows_;
            o.bcsr_row_ptr_ = nullptr;
            o.bcsr_col_ind_ = nullptr;
            o.bcsr_values_ = nullptr;
            o.dispatch_order_ = nullptr;
        }
        return *this;
    }

    IndexType get_num_block_rows() const { return num_block_rows_; }
    IndexType get_num_block_cols() const { return num_block_cols_; }
    IndexType get_num_blocks() const { return num_blocks_; }
    IndexType get_r_block() const { return r_block_; }
    IndexType get_c_block() const { return c_block_; }

    // Element shape (see the header comment).
    IndexType get_num_rows() const { return num_rows_; }
    IndexType get_num_cols() const { return num_cols_; }
    void set_shape(IndexType num_rows, IndexType num_cols) {
        if (num_rows < 0 || num_cols < 0 || num_rows > num_block_rows_ * r_block_ ||
            num_cols > num_block_cols_ * c_block_) {
            throw std::invalid_argument("BCSR element shape exceeds its block grid.");
        }
        num_rows_ = num_rows;
        num_cols_ = num_cols;
    }

    IndexType* get_bcsr_row_ptr() const { return bcsr_row_ptr_; }
    IndexType* get_bcsr_col_ind() const { return bcsr_col_ind_; }
    ValueType* get_bcsr_values() const { return bcsr_values_; }

    std::shared_ptr<const Executor> get_executor() const { return exec_; }

    // Dispatch order of the Tier-1 column-batch kernels (block-row ids; at
    // least num_block_rows int32 entries on the executor), which csr_to_bcsr
    // computes once per matrix so that Tier-1 calls do not order the rows
    // again: above 2048 block-rows the longest rows first, from 256 a
    // contiguous range of block-rows per XCD when the rows are short and
    // neighbouring rows alike.  Null: Tier-1 orders the rows on each call
    // when it needs to (above 2048 block-rows).  set_dispatch_order takes ownership of an array allocated
    // with this matrix's executor; copy_from_host drops it (the row lengths
    // may change).
    const int32_t* get_dispatch_order() const { return dispatch_order_; }
    void set_dispatch_order(int32_t* order)
    {
        free_dispatch_order();
        dispatch_order_ = order;
    }

    // Whether Tier-1 (fp16) takes the band kernel for this matrix: every
    // block-row one contiguous run of block columns, and four neighbouring
    // block-rows sharing B tiles gather fewer B rows than the column-batch
    // kernel would.  csr_to_bcsr decides it once per matrix; the band kernel
    // is only correct on contiguous rows, so set it only from that check.
    // copy_from_host clears it.
    bool get_band_rows() const { return band_rows_; }
    void set_band_rows(bool band) { band_rows_ = band; }

    void copy_from_host(const IndexType* host_row_ptr, const IndexType* host_col_ind,
                        const ValueType* host_values)
    {
        free_dispatch_order();
        band_rows_ = false;
        exec_->copy_from_host(bcsr_row_ptr_, host_row_ptr,
                              (static_cast<size_t>(num_block_rows_) + 1) * sizeof(IndexType));
        if (num_blocks_ > 0) {
            exec_->copy_from_host(bcsr_col_ind_, host_col_ind,
                                  static_cast<size_t>(num_blocks_) * sizeof(IndexType));
            exec_->copy_from_host(bcsr_values_, host_values, value_bytes());
        }
    }

private:
    size_t value_bytes() const {
        return static_cast<size_t>(num_blocks_) * static_cast<size_t>(r_block_) *
               static_cast<size_t>(c_block_) * sizeof(ValueType);
    }

    void free_dispatch_order() noexcept {
        if (exec_ && dispatch_order_) {
            try {
                exec_->free(dispatch_order_);
            } catch (...) {
            }
        }
        dispatch_order_ = nullptr;
    }

    void release() noexcept {
        if (!exec_) return;
        free_dispatch_order();
        try {
            if (bcsr_row_ptr_) exec_->free(bcsr_row_ptr_);
            if (bcsr_col_ind_) exec_->free(bcsr_col_ind_);
            if (bcsr_values_) exec_->free(bcsr_values_);
        } catch (...) {
        }
        bcsr_row_ptr_ = nullptr;
        bcsr_col_ind_ = nullptr;
        bcsr_values_ = nullptr;
    }

    std::shared_ptr<const Executor> exec_;
    IndexType num_block_rows_;
    IndexType num_block_cols_;
    IndexType num_blocks_;
    IndexType r_block_;
    IndexType c_block_;
    IndexType num_rows_;
    IndexType num_cols_;

    IndexType* bcsr_row_ptr_ = nullptr;
    IndexType* bcsr_col_ind_ = nullptr;
    ValueType* bcsr_values_ = nullptr;
    int32_t* dispatch_order_ = nullptr;
    bool band_rows_ = false;
};

}  // namespace xspmm
