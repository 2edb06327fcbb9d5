// rhizome_delta_grad.hpp -- the adjoint of the gated delta rule, in f64 on
// the CPU, and the finite-difference gradient check it is held to.
//
// The reference names the adjoint ("reverse scan of the rank-1 update",
// docs/kernels.md:16) but has no implementation; the forward it inverts is
// gated_delta_step / gated_delta_sequential (crates/ops/src/delta.rs:94-154).
// Backward passes stay on the CPU, so this is host code with no GPU path.
//
// For one position, with P the state entering it (zero after a reset),
// sk = P k, S = alpha (P - beta sk k^T) + beta v k^T and o = S q, and with
// dS the gradient reaching S (from o, from later positions and from the
// final state):
//
//   dS    += do q^T                       dq     = S^T do
//   w      = dS k
//   dv     = beta w                       dalpha = <dS, P> - beta sk.w
//   dbeta  = (v - alpha sk).w
//   dk     = dS^T (beta v - alpha beta sk) - alpha beta P^T w
//   dP     = alpha (dS - beta w k^T)      (cut to zero across a reset)
//
// The reverse scan needs every entering state.  The forward is re-run once
// and the state is kept every 64 positions; each 64-position window is then
// re-run from its checkpoint, so memory is O((T / 64 + 64) d_v d_k), not
// O(T d_v d_k).
//
//   gated_delta_sequential_backward  delta.rs:133-154's signature: one head,
//                                    square state, reset at t = 0 and at
//                                    every segment change
//   gated_delta_prefill_backward     the batched prefill of rhz_gdr_prefill
//                                    (include/rhizome_gdr.h): packed
//                                    sequences, H heads, d_v x d_k state,
//                                    initial state honoured, alpha or
//                                    log-decay gates, threads over (seq, head)
//   gradcheck::check                 crates/ops/src/gradcheck.rs:3-53
#pragma once

#include <cstddef>
#include <cstdint>
#include <functional>
#include <vector>

#include "rhizome_delta.hpp"

namespace rhizome {
namespace ops {

// Gradients of a scalar loss with respect to every input of the forward.
struct DeltaGrads {
    std::vector<double> q, k, v;   // T x head_dim
    std::vector<double> alpha, beta;
    DeltaState init;               // nonzero only for an empty sequence (t = 0 resets)
};

// Adjoint of gated_delta_sequential(inp, init): d_out is dL/do (T x head_dim),
// d_final dL/d(final state) (nullptr for zero).  Throws Error where the
// forward would panic.
DeltaGrads gated_delta_sequential_backward(const DeltaInputs& inp, const DeltaState& init,
                                           const std::vector<double>& d_out, const DeltaState* d_final = nullptr);

// Batched adjoint of the prefill: layouts as rhz_gdr_prefill_args, in f64.
struct PrefillBackwardArgs {
    int32_t batch = 0;    // dense: B; packed: number of sequences N
    int32_t seq_len = 0;  // dense: T; packed: total tokens
    int32_t heads = 0, d_k = 0, d_v = 0;
    int32_t gate_kind = 0;              // rhz_gate: 0 log-decay g (alpha = exp g), 1 alpha
    const double* q = nullptr;          // [tokens, H, d_k]
    const double* k = nullptr;          // [tokens, H, d_k]
    const double* v = nullptr;          // [tokens, H, d_v]
    const double* gate = nullptr;       // [tokens, H]
    const double* beta = nullptr;       // [tokens, H]
    const int64_t* cu_seqlens = nullptr;     // [N + 1] token offsets, or nullptr for dense
    const double* initial_state = nullptr;   // [batch, H, d_v, d_k], or nullptr for zeros
    const double* d_o = nullptr;             // [tokens, H, d_v]
    const double* d_final_state = nullptr;   // [batch, H, d_v, d_k], or nullptr for zero
    double* dq = nullptr;                    // outputs, same layouts as the inputs
    double* dk = nullptr;
    double* dv = nullptr;
    double* dgate = nullptr;
    double* dbeta = nullptr;
    double* d_initial_state = nullptr;       // may be nullptr
    int threads = 0;                          // 0: hardware concurrency
};

void gated_delta_prefill_backward(const PrefillBackwardArgs& a);

namespace gradcheck {

// (f(x + h e_i) - f(x - h e_i)) / 2h with h = 1e-5 (gradcheck.rs:3-14).
double central_difference(const std::function<double(const std::vector<double>&)>& f, const std::vector<double>& x,
                          std::size_t i);

struct GradCheckReport {
    double max_rel_err = 0.0;
    std::size_t worst_index = 0;
    bool passes(double rtol) const { return max_rel_err <= rtol; }
};

// Largest |fd - analytic| / max(|fd|, |analytic|, 1e-6) over every
// coordinate (gradcheck.rs:33-53).
GradCheckReport check(const std::function<double(const std::vector<double>&)>& f, const std::vector<double>& x,
                      const std::vector<double>& analytic);

}  // namespace gradcheck
}  // namespace ops
}  // namespace rhizome
