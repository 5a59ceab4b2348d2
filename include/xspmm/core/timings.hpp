#pragma once

namespace xspmm {

// Per-stage wall times of the Tier-2 pipeline, in milliseconds.
// Same fields and defaults as the reference (include/xspmm/core/timings.hpp:7-14).
// Fields of stages a call does not run keep the caller's values.
struct SpMMTimings {
    double clustering_ms = 0.0;
    double permutation_ms = 0.0;
    double conversion_ms = 0.0;
    double spmm_ms = 0.0;
    double unpermutation_ms = 0.0;
    double total_pipeline_ms = 0.0;
};

}  // namespace xspmm
