// rhizome_delta.hpp -- the gated delta-rule API of crates/ops/src/delta.rs,
// restated in C++ over librhizome_gdr.so (MI355X), so that a host caller of
// the reference finds the same types, names, argument meaning and results.
//
//   DeltaInputs             delta.rs:12-56
//   DeltaState              delta.rs:58-90
//   gated_delta_step        delta.rs:92-127
//   gated_delta_sequential  delta.rs:129-154
//   gated_delta_scan_chunked delta.rs:156-197
//   gated_delta_multistep   delta.rs:199-230
//
// Values cross to the GPU as fp32 and come back widened to f64: results
// agree with the f64 reference to fp32 accuracy (relative 1e-4), not
// bitwise.  Each call copies its inputs to device memory and its results
// back, so this API suits migration and testing; batched device-resident
// callers use include/rhizome_gdr.h directly.
//
// Errors: where the reference panics (inconsistent lengths, delta.rs slice
// indexing), these functions throw rhizome::ops::Error before any GPU work;
// a library or HIP failure also throws Error, with the library's status and
// message.
#pragma once

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "rhizome_error.hpp"

namespace rhizome {
namespace ops {

// Per-position inputs for one head (delta.rs:12-29): rows T x head_dim,
// alpha in (0, 1], beta in (0, 1), and a segment id per position (a change
// resets the state).
struct DeltaInputs {
    std::size_t head_dim = 0;
    std::vector<double> q, k, v;
    std::vector<double> alpha, beta;
    std::vector<std::size_t> segment;

    std::size_t len() const { return alpha.size(); }
    bool is_empty() const { return len() == 0; }
    // delta.rs:46-55: every length agrees with len() and head_dim > 0.
    bool is_consistent() const;
};

// Recurrent state of one head, row-major S[i][j] at i * head_dim + j
// (i = value row, j = key column; delta.rs:58-65).
struct DeltaState {
    std::size_t head_dim = 0;
    std::vector<double> s;

    static DeltaState zeros(std::size_t head_dim);
    void reset();
    double max_abs_diff(const DeltaState& other) const;
};

// One position, state updated in place; returns o_t (delta.rs:94-127).
std::vector<double> gated_delta_step(DeltaState& state, const std::vector<double>& q,
                                     const std::vector<double>& k, const std::vector<double>& v,
                                     double alpha, double beta);

// Whole sequence; returns (o, final state) (delta.rs:133-154).  As in the
// reference, the state is reset at t = 0 and at every segment change, so
// `init` only matters for an empty sequence (it is then returned).
std::pair<std::vector<double>, DeltaState> gated_delta_sequential(const DeltaInputs& inp,
                                                                  const DeltaState& init);

// Same result for every chunk >= 1 (delta.rs:156-197).
std::pair<std::vector<double>, DeltaState> gated_delta_scan_chunked(const DeltaInputs& inp,
                                                                    const DeltaState& init,
                                                                    std::size_t chunk);

// The first min(T, max_positions) positions with the state after each
// (delta.rs:202-230); reset at t = 0 and at segment changes.
std::pair<std::vector<double>, std::vector<DeltaState>> gated_delta_multistep(const DeltaInputs& inp,
                                                                             const DeltaState& init,
                                                                             std::size_t max_positions);

}  // namespace ops
}  // namespace rhizome
