// rhizome_plan.hpp -- the plan-level IR of crates/plan restated in C++: the
// element formats a tensor declaration names, the closed op vocabulary, the
// SSA graph and the arena planner, so that a plan built here is the plan the
// reference builds for the same graph (same intervals, offsets and size).
//
//   DType, bytes_for        crates/core/src/dtype.rs:5-55
//   OpKind, name            crates/plan/src/graph.rs:35-84, 111-139
//   TensorDesc, Node, Graph crates/plan/src/graph.rs:142-293
//   Interval, ArenaPlan     crates/plan/src/arena.rs:6-67
//   kAlign, plan            crates/plan/src/arena.rs:70-144
//
// Errors are rhizome::Error with RHZ_ERR_INVALID_ARG where the reference
// returns Error::Shape.  The executor over a plan is rhizome_exec.hpp.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

#include "rhizome_error.hpp"

namespace rhizome {
namespace plan {

// Tensor element formats (dtype.rs:5-20).
enum class DType { F64, F32, BF16, F8E4M3, MXFP4, MXINT4, I8 };

// Bits per element, excluding block scales (dtype.rs:32-40).
std::size_t bits(DType d);
// Elements sharing one e8m0 scale, 1 for unblocked formats (dtype.rs:24-29).
std::size_t block_size(DType d);
// Bytes for n elements: payload rounded up to whole bytes, plus one scale
// byte per block for the MX formats (dtype.rs:44-55).
std::size_t bytes_for(DType d, std::size_t n);
const char* dtype_name(DType d);

// The closed op vocabulary (graph.rs:35-84), in the reference's order.
enum class OpKind {
    Add,
    Mul,
    Silu,
    Swiglu,
    ResidualAdd,
    RmsNorm,
    Linear,
    GroupedLinear,
    Softmax,
    DeltaScan,
    DeltaStep,
    MlaCompress,
    MlaPrefill,
    MlaDecode,
    RouterTopk,
    MoePermute,
    MoeUnpermute,
    PkmLookup,
    CrossEntropyZLoss,
    HaltHead,
    Sample,
    QuantizeMx,
    AllReduce,
};

// Stable op name (graph.rs:111-139), e.g. "gated_delta_scan_chunked".
const char* name(OpKind op);

using TensorId = std::size_t;

struct TensorDesc {
    std::string name;
    std::size_t elems = 0;
    DType dtype = DType::F32;
    bool is_param = false;  // parameters live outside the arena
    std::size_t bytes() const { return bytes_for(dtype, elems); }
};

struct Node {
    OpKind op;
    std::vector<TensorId> inputs;
    TensorId output;
};

// A directed acyclic graph in insertion (topological) order.
class Graph {
public:
    // Declare a tensor; returns its id.
    TensorId tensor(const std::string& name, std::size_t elems, DType dtype, bool is_param);
    // Append a node writing a freshly declared tensor; throws for an unknown
    // input id (graph.rs:199-220).
    TensorId push(OpKind op, const std::vector<TensorId>& inputs, const std::string& out_name,
                  std::size_t out_elems, DType out_dtype);
    const std::vector<Node>& nodes() const { return nodes_; }
    const std::vector<TensorDesc>& tensors() const { return tensors_; }
    const TensorDesc& desc(TensorId id) const;  // throws for an unknown id
    // SSA outputs, defined-before-use, no parameter written (graph.rs:252-293).
    void validate() const;

private:
    std::vector<TensorDesc> tensors_;
    std::vector<Node> nodes_;
};

// Live range of one tensor in node indices (inclusive) and its arena bytes.
struct Interval {
    TensorId tensor = 0;
    std::size_t start = 0, end = 0;
    std::size_t offset = 0, size = 0;
    bool overlaps_time(const Interval& o) const { return start <= o.end && o.start <= end; }
    bool overlaps_memory(const Interval& o) const {
        return offset < o.offset + o.size && o.offset < offset + size;
    }
};

struct ArenaPlan {
    std::vector<Interval> intervals;  // ordered by tensor id
    std::size_t total_bytes = 0;
    // Throws when two tensors live at the same time share arena bytes
    // (arena.rs:49-61).
    void verify() const;
    // Bytes if every tensor had its own allocation (arena.rs:63-67).
    std::size_t unplanned_bytes() const;
    // The interval of a tensor, or nullptr when it is not in the arena.
    const Interval* find(TensorId t) const;
};

constexpr std::size_t kAlign = 256;  // arena.rs:71

// Liveness over node indices, then greedy placement, largest tensor first
// (ties by id): walk the byte ranges of the tensors already placed that are
// live at the same time, in address order, and take the first gap the
// tensor's 256-byte-rounded size fits in, else the end of the last range
// (arena.rs:83-144).  Parameters are excluded.
//
// pin_boundary = false reproduces the reference exactly.  pin_boundary = true
// is the executor's liveness: every graph input (a tensor no node writes)
// and graph output (a tensor no node reads) is live from node 0 to the last
// node, so that a caller can write every input before a run and read every
// output -- and every state updated in place -- after it; the placement rule
// is the same.
ArenaPlan plan(const Graph& graph, bool pin_boundary = false);

}  // namespace plan
}  // namespace rhizome
