// rhizome_plan.cpp -- crates/plan's graph IR and arena planner in C++.

#include "rhizome_plan.hpp"

#include <algorithm>
#include <limits>
#include <set>
#include <tuple>
#include <utility>

#include "rhizome_gdr.h"

namespace rhizome {
namespace plan {
namespace {

[[noreturn]] void shape_error(const std::string& what) { throw Error(RHZ_ERR_INVALID_ARG, what); }

std::size_t align_up(std::size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

}  // namespace

std::size_t bits(DType d) {
    switch (d) {
        case DType::F64: return 64;
        case DType::F32: return 32;
        case DType::BF16: return 16;
        case DType::F8E4M3:
        case DType::I8: return 8;
        case DType::MXFP4:
        case DType::MXINT4: return 4;
    }
    return 0;
}

std::size_t block_size(DType d) { return d == DType::MXFP4 || d == DType::MXINT4 ? 32 : 1; }

std::size_t bytes_for(DType d, std::size_t n) {
    const std::size_t payload = (n * bits(d) + 7) / 8;
    const std::size_t block = block_size(d);
    return block > 1 ? payload + (n + block - 1) / block : payload;
}

const char* dtype_name(DType d) {
    switch (d) {
        case DType::F64: return "f64";
        case DType::F32: return "f32";
        case DType::BF16: return "bf16";
        case DType::F8E4M3: return "f8e4m3";
        case DType::MXFP4: return "mxfp4";
        case DType::MXINT4: return "mxint4";
        case DType::I8: return "i8";
    }
    return "?";
}

const char* name(OpKind op) {
    switch (op) {
        case OpKind::Add: return "add";
        case OpKind::Mul: return "mul";
        case OpKind::Silu: return "silu";
        case OpKind::Swiglu: return "swiglu";
        case OpKind::ResidualAdd: return "residual_add";
        case OpKind::RmsNorm: return "rmsnorm";
        case OpKind::Linear: return "linear";
        case OpKind::GroupedLinear: return "grouped_linear";
        case OpKind::Softmax: return "softmax";
        case OpKind::DeltaScan: return "gated_delta_scan_chunked";
        case OpKind::DeltaStep: return "gated_delta_step";
        case OpKind::MlaCompress: return "mla_compress";
        case OpKind::MlaPrefill: return "mla_prefill";
        case OpKind::MlaDecode: return "mla_decode";
        case OpKind::RouterTopk: return "router_topk_grouped";
        case OpKind::MoePermute: return "moe_permute";
        case OpKind::MoeUnpermute: return "moe_unpermute";
        case OpKind::PkmLookup: return "pkm_gather_sum";
        case OpKind::CrossEntropyZLoss: return "cross_entropy_zloss";
        case OpKind::HaltHead: return "halt_head";
        case OpKind::Sample: return "sampling";
        case OpKind::QuantizeMx: return "quantize_mx";
        case OpKind::AllReduce: return "all_reduce";
    }
    return "?";
}

TensorId Graph::tensor(const std::string& name, std::size_t elems, DType dtype, bool is_param) {
    tensors_.push_back(TensorDesc{name, elems, dtype, is_param});
    return tensors_.size() - 1;
}

TensorId Graph::push(OpKind op, const std::vector<TensorId>& inputs, const std::string& out_name,
                     std::size_t out_elems, DType out_dtype) {
    for (TensorId i : inputs)
        if (i >= tensors_.size()) shape_error("unknown input tensor " + std::to_string(i));
    const TensorId out = tensor(out_name, out_elems, out_dtype, false);
    nodes_.push_back(Node{op, inputs, out});
    return out;
}

const TensorDesc& Graph::desc(TensorId id) const {
    if (id >= tensors_.size()) shape_error("unknown tensor " + std::to_string(id));
    return tensors_[id];
}

void Graph::validate() const {
    std::set<TensorId> written;
    for (const Node& n : nodes_) written.insert(n.output);
    // Parameters and tensors no node writes are defined before node 0.
    std::set<TensorId> live;
    for (TensorId i = 0; i < tensors_.size(); ++i)
        if (tensors_[i].is_param || !written.count(i)) live.insert(i);
    std::set<TensorId> seen_outputs;
    for (std::size_t idx = 0; idx < nodes_.size(); ++idx) {
        const Node& n = nodes_[idx];
        for (TensorId i : n.inputs)
            if (!live.count(i))
                shape_error("node " + std::to_string(idx) + " (" + name(n.op) + ") uses tensor " +
                            std::to_string(i) + " before it is defined");
        if (!seen_outputs.insert(n.output).second)
            shape_error("tensor " + std::to_string(n.output) + " is written more than once (SSA violation)");
        if (n.output >= tensors_.size()) shape_error("unknown tensor " + std::to_string(n.output));
        if (tensors_[n.output].is_param)
            shape_error("node " + std::to_string(idx) + " writes parameter tensor " + std::to_string(n.output));
        live.insert(n.output);
    }
}

void ArenaPlan::verify() const {
    for (std::size_t i = 0; i < intervals.size(); ++i)
        for (std::size_t j = i + 1; j < intervals.size(); ++j) {
            const Interval& a = intervals[i];
            const Interval& b = intervals[j];
            if (a.overlaps_time(b) && a.overlaps_memory(b))
                shape_error("tensors " + std::to_string(a.tensor) + " and " + std::to_string(b.tensor) +
                            " are live together but share arena bytes");
        }
}

std::size_t ArenaPlan::unplanned_bytes() const {
    std::size_t s = 0;
    for (const Interval& i : intervals) s += i.size;
    return s;
}

const Interval* ArenaPlan::find(TensorId t) const {
    for (const Interval& i : intervals)
        if (i.tensor == t) return &i;
    return nullptr;
}

ArenaPlan plan(const Graph& graph, bool pin_boundary) {
    const auto& tensors = graph.tensors();
    const auto& nodes = graph.nodes();
    const std::size_t n = tensors.size();
    std::vector<std::size_t> start(n, std::numeric_limits<std::size_t>::max()), end(n, 0);
    std::vector<char> used(n, 0), read(n, 0), written(n, 0);
    auto touch = [&](TensorId i, std::size_t idx) {
        used[i] = 1;
        start[i] = std::min(start[i], idx);
        end[i] = std::max(end[i], idx);
    };
    for (std::size_t idx = 0; idx < nodes.size(); ++idx) {
        const Node& node = nodes[idx];
        for (TensorId i : node.inputs) {
            if (graph.desc(i).is_param) continue;
            read[i] = 1;
            touch(i, idx);
        }
        graph.desc(node.output);
        written[node.output] = 1;
        touch(node.output, idx);
    }
    if (pin_boundary && !nodes.empty())
        for (TensorId i = 0; i < n; ++i)
            if (used[i] && (!written[i] || !read[i])) {
                start[i] = 0;
                end[i] = nodes.size() - 1;
            }

    std::vector<TensorId> order;
    for (TensorId i = 0; i < n; ++i)
        if (used[i] && !tensors[i].is_param) order.push_back(i);
    // Largest first, ties by id.
    std::sort(order.begin(), order.end(), [&](TensorId a, TensorId b) {
        const std::size_t ba = tensors[a].bytes(), bb = tensors[b].bytes();
        return ba != bb ? ba > bb : a < b;
    });

    std::vector<Interval> placed;
    for (TensorId id : order) {
        Interval cand;
        cand.tensor = id;
        cand.start = start[id];
        cand.end = end[id];
        cand.size = align_up(std::max<std::size_t>(tensors[id].bytes(), 1));
        // Byte ranges of the tensors placed so far that are live together.
        std::vector<std::pair<std::size_t, std::size_t>> blocks;
        for (const Interval& p : placed)
            if (p.overlaps_time(cand)) blocks.emplace_back(p.offset, p.offset + p.size);
        std::sort(blocks.begin(), blocks.end());
        std::size_t offset = 0;
        for (const auto& [lo, hi] : blocks) {
            if (offset + cand.size <= lo) break;
            offset = std::max(offset, hi);
        }
        cand.offset = offset;
        placed.push_back(cand);
    }
    std::sort(placed.begin(), placed.end(), [](const Interval& a, const Interval& b) { return a.tensor < b.tensor; });
    ArenaPlan out;
    for (const Interval& i : placed) out.total_bytes = std::max(out.total_bytes, i.offset + i.size);
    out.intervals = std::move(placed);
    out.verify();
    return out;
}

}  // namespace plan
}  // namespace rhizome
