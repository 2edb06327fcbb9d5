// rhizome_exec.hpp -- an executor for plans (rhizome_plan.hpp) on MI355X:
// the arena of an ArenaPlan becomes one device allocation, every tensor in it
// a 256-byte-aligned offset into that allocation, and the nodes run in order
// on one HIP stream through librhizome_gdr.so.
//
// The reference plans graphs (crates/plan/src/arena.rs:83-144) but has no
// executor; the op identities it would dispatch on are
// OpKind::DeltaScan / DeltaStep (crates/plan/src/graph.rs:56-59).  This one
// runs:
//
//   DeltaScan  inputs [q, k, v, gate, beta] or [q, k, v, gate, beta, state],
//              output o.  q, k [tokens, H, d_k], v and o [tokens, H, d_v] in
//              F32 or BF16; gate, beta F32 [tokens, H]; state F32
//              [sequences, H, d_v, d_k], read as the initial state and
//              overwritten with the final one.  Without a state operand the
//              scan starts from zeros and the final state is dropped, as
//              gated_delta_scan_chunked resets at t = 0 (delta.rs:159-197).
//   DeltaStep  inputs [q, k, v, gate, beta, state], output o; q, k [B, H, d_k],
//              v and o [B, H, d_v], gate and beta [B, H]; the F32 state
//              [B, H, d_v, d_k] is updated in place, as gated_delta_step
//              takes &mut DeltaState (delta.rs:94-127).
//   RmsNorm    inputs [x, scale], output y; x and y [rows, dim] in F32 or BF16,
//              scale F32 [dim] (crates/ops/src/norm.rs:8-13, per row).
//
// A graph node carries no shapes (graph.rs:163-171), so each dispatched node
// gets its shapes from an attribute record.  compile() is the plan-time
// check (R4, SPEC.md:28-30): every node must be one of the three ops above,
// with its attributes, operand count, element counts and formats agreeing
// and (op, dtype, d_k, d_v) supported by the library; anything else throws
// rhizome::Error (RHZ_ERR_UNSUPPORTED for an op or shape the library does
// not run, RHZ_ERR_INVALID_ARG for an inconsistent graph) before any device
// memory is touched.
//
// Memory: the arena plan (rhizome::plan::plan with pin_boundary = true, so
// graph inputs and outputs stay live through the whole run), followed by the
// packed-sequence offsets of every DeltaScan node and one prefill workspace
// sized for the largest DeltaScan, all in one hipMalloc.  Parameters and
// state caches may instead live outside the arena (TensorDesc::is_param):
// the caller binds their device addresses.  The library itself allocates
// nothing, so a run can also be captured once as a HIP graph and replayed.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <map>
#include <variant>
#include <vector>

#include "rhizome_gdr.h"
#include "rhizome_plan.hpp"

namespace rhizome {
namespace exec {

using plan::TensorId;

struct DeltaScanAttrs {
    int32_t batch = 0;    // dense: B; packed: number of sequences N
    int32_t seq_len = 0;  // dense: T; packed: total tokens
    int32_t heads = 0, d_k = 0, d_v = 0;
    int32_t chunk = 64;   // the result does not depend on it (delta.rs:156-157)
    int32_t gate_kind = RHZ_GATE_LOG_ALPHA;
    int32_t algo = RHZ_ALGO_AUTO;
    std::vector<int32_t> cu_seqlens;  // empty: dense; else N + 1 offsets from 0 to seq_len
};

struct DeltaStepAttrs {
    int32_t batch = 0, heads = 0, d_k = 0, d_v = 0;
    int32_t gate_kind = RHZ_GATE_LOG_ALPHA;
};

struct RmsNormAttrs {
    int32_t rows = 0, dim = 0;
    float eps = 1e-6f;
};

using NodeAttrs = std::variant<DeltaScanAttrs, DeltaStepAttrs, RmsNormAttrs>;

// The checked plan: where every tensor lives and what each node launches.
class CompiledPlan {
public:
    const plan::Graph& graph() const { return graph_; }
    const plan::ArenaPlan& arena() const { return arena_; }
    // Bytes of the one device allocation: arena, sequence offsets, workspace.
    std::size_t device_bytes() const { return device_bytes_; }
    std::size_t workspace_bytes() const { return workspace_bytes_; }
    // Offset of a tensor in the device allocation; throws for a parameter
    // or a tensor no node uses.
    std::size_t offset(TensorId t) const;

private:
    friend CompiledPlan compile(const plan::Graph&, const std::map<std::size_t, NodeAttrs>&);
    friend class Executor;
    struct Step {
        std::size_t node;
        NodeAttrs attrs;
        std::size_t cu_offset;  // of its packed-sequence offsets, if any
    };
    plan::Graph graph_;
    plan::ArenaPlan arena_;
    std::vector<Step> steps_;
    std::size_t cu_base_ = 0, workspace_offset_ = 0, workspace_bytes_ = 0, device_bytes_ = 0;
};

// Validate the graph, check every node against its attributes and the
// library's capabilities, and lay out device memory.  attrs maps a node
// index to its attributes.  Makes no HIP call that touches a device.
CompiledPlan compile(const plan::Graph& graph, const std::map<std::size_t, NodeAttrs>& attrs);

class Executor {
public:
    // One hipMalloc of plan.device_bytes() on the current device, zeroed,
    // with the packed-sequence offsets copied in.
    explicit Executor(CompiledPlan plan);
    ~Executor();
    Executor(const Executor&) = delete;
    Executor& operator=(const Executor&) = delete;

    // The device address of a parameter (is_param) tensor.  Every parameter
    // a node reads must be bound before run().
    void bind(TensorId param, void* device_ptr);
    // Device address of a tensor: arena base + offset, or its binding.
    void* data(TensorId t) const;
    // Launch every node in order on `stream` (asynchronous).
    void run(hipStream_t stream = nullptr);
    // Record run() on `stream` into a HIP graph once; replay() launches it.
    // Bindings are captured by value: bind again, then capture again.
    void capture(hipStream_t stream);
    void replay(hipStream_t stream = nullptr);

    const CompiledPlan& plan() const { return plan_; }
    void* base() const { return base_; }

private:
    CompiledPlan plan_;
    void* base_ = nullptr;
    std::map<TensorId, void*> bound_;
    hipGraph_t graph_ = nullptr;
    hipGraphExec_t graph_exec_ = nullptr;
    void release_graph();
};

}  // namespace exec
}  // namespace rhizome
