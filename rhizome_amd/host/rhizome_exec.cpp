// rhizome_exec.cpp -- plan-time checks, device layout and dispatch of a plan
// through librhizome_gdr.so.

#include "rhizome_exec.hpp"

#include <algorithm>
#include <string>
#include <utility>

namespace rhizome {
namespace exec {
namespace {

using plan::DType;
using plan::OpKind;

std::size_t align_up(std::size_t x) { return (x + plan::kAlign - 1) / plan::kAlign * plan::kAlign; }

std::string where(std::size_t idx, const plan::Node& n) {
    return "node " + std::to_string(idx) + " (" + plan::name(n.op) + ")";
}

[[noreturn]] void invalid(const std::string& what) { throw Error(RHZ_ERR_INVALID_ARG, what); }

void check_status(int32_t status, const std::string& what) {
    if (status != RHZ_OK) throw Error(status, what + ": " + rhz_status_string(status) + ": " + rhz_last_error());
}

void hip_check(hipError_t e, const char* call) {
    if (e != hipSuccess) throw Error(RHZ_ERR_HIP, std::string(call) + ": " + hipGetErrorString(e));
}

int32_t act_dtype(DType d, const std::string& at) {
    if (d == DType::F32) return RHZ_F32;
    if (d == DType::BF16) return RHZ_BF16;
    throw Error(RHZ_ERR_UNSUPPORTED, at + ": activations must be f32 or bf16, not " + plan::dtype_name(d));
}

// Operand `slot` of a node must hold `elems` elements of `dtype`.
void expect(const plan::Graph& g, TensorId id, std::size_t elems, DType dtype, const char* slot,
            const std::string& at) {
    const plan::TensorDesc& t = g.desc(id);
    if (t.elems != elems || t.dtype != dtype)
        invalid(at + ": " + slot + " '" + t.name + "' holds " + std::to_string(t.elems) + " " +
                plan::dtype_name(t.dtype) + " elements, expected " + std::to_string(elems) + " " +
                plan::dtype_name(dtype));
}

void positive(int64_t v, const char* what, const std::string& at) {
    if (v < 1) invalid(at + ": " + what + " must be >= 1 (got " + std::to_string(v) + ")");
}

// DeltaScan: shapes, packed offsets, capability, workspace bytes.
std::size_t check_scan(const plan::Graph& g, const plan::Node& n, const DeltaScanAttrs& a, const std::string& at) {
    if (n.inputs.size() != 5 && n.inputs.size() != 6)
        invalid(at + ": takes [q, k, v, gate, beta] or [q, k, v, gate, beta, state], got " +
                std::to_string(n.inputs.size()) + " inputs");
    positive(a.batch, "batch", at);
    positive(a.heads, "heads", at);
    positive(a.d_k, "d_k", at);
    positive(a.d_v, "d_v", at);
    if (a.seq_len < 0) invalid(at + ": seq_len must be >= 0");
    const bool packed = !a.cu_seqlens.empty();
    if (packed) {
        if (a.cu_seqlens.size() != static_cast<std::size_t>(a.batch) + 1)
            invalid(at + ": cu_seqlens holds " + std::to_string(a.cu_seqlens.size()) + " offsets, expected batch + 1 = " +
                    std::to_string(a.batch + 1));
        if (a.cu_seqlens.front() != 0 || a.cu_seqlens.back() != a.seq_len)
            invalid(at + ": cu_seqlens must run from 0 to seq_len");
        for (std::size_t i = 1; i < a.cu_seqlens.size(); ++i)
            if (a.cu_seqlens[i] < a.cu_seqlens[i - 1]) invalid(at + ": cu_seqlens must be non-decreasing");
    }
    const int32_t dt = act_dtype(g.desc(n.inputs[0]).dtype, at);
    check_status(rhz_gdr_query_support(RHZ_OP_DELTA_SCAN, dt, a.d_k, a.d_v, a.algo), at);

    rhz_gdr_prefill_args pa{};
    pa.batch = a.batch;
    pa.seq_len = a.seq_len;
    pa.heads = a.heads;
    pa.d_k = a.d_k;
    pa.d_v = a.d_v;
    pa.chunk = a.chunk;
    pa.dtype = dt;
    pa.gate_kind = a.gate_kind;
    pa.algo = a.algo;
    // Only presence matters to the size query; it reads no pointer.
    static const int32_t kPresent = 0;
    pa.cu_seqlens = packed ? &kPresent : nullptr;
    std::size_t ws = 0;
    // Also bounds every dimension and index range.
    check_status(rhz_gdr_prefill_workspace_size(&pa, &ws), at);

    const std::size_t tokens = packed ? std::size_t(a.seq_len) : std::size_t(a.batch) * a.seq_len;
    const std::size_t H = a.heads, dk = a.d_k, dv = a.d_v;
    const DType act = g.desc(n.inputs[0]).dtype;
    expect(g, n.inputs[0], tokens * H * dk, act, "q", at);
    expect(g, n.inputs[1], tokens * H * dk, act, "k", at);
    expect(g, n.inputs[2], tokens * H * dv, act, "v", at);
    expect(g, n.inputs[3], tokens * H, DType::F32, "gate", at);
    expect(g, n.inputs[4], tokens * H, DType::F32, "beta", at);
    if (n.inputs.size() == 6) expect(g, n.inputs[5], std::size_t(a.batch) * H * dv * dk, DType::F32, "state", at);
    expect(g, n.output, tokens * H * dv, act, "o", at);

    return ws;
}

void check_step(const plan::Graph& g, const plan::Node& n, const DeltaStepAttrs& a, const std::string& at) {
    if (n.inputs.size() != 6) invalid(at + ": takes [q, k, v, gate, beta, state], got " + std::to_string(n.inputs.size()) + " inputs");
    positive(a.batch, "batch", at);
    positive(a.heads, "heads", at);
    positive(a.d_k, "d_k", at);
    positive(a.d_v, "d_v", at);
    if (a.gate_kind != RHZ_GATE_LOG_ALPHA && a.gate_kind != RHZ_GATE_ALPHA) invalid(at + ": unknown gate_kind");
    const int32_t dt = act_dtype(g.desc(n.inputs[0]).dtype, at);
    check_status(rhz_gdr_query_support(RHZ_OP_DELTA_STEP, dt, a.d_k, a.d_v, RHZ_ALGO_AUTO), at);
    if (int64_t(a.batch) * a.heads * a.d_v * a.d_k >= (int64_t(1) << 40))
        invalid(at + ": batch * heads * d_v * d_k exceeds 2^40");
    const std::size_t BH = std::size_t(a.batch) * a.heads, dk = a.d_k, dv = a.d_v;
    const DType act = g.desc(n.inputs[0]).dtype;
    expect(g, n.inputs[0], BH * dk, act, "q", at);
    expect(g, n.inputs[1], BH * dk, act, "k", at);
    expect(g, n.inputs[2], BH * dv, act, "v", at);
    expect(g, n.inputs[3], BH, DType::F32, "gate", at);
    expect(g, n.inputs[4], BH, DType::F32, "beta", at);
    expect(g, n.inputs[5], BH * dv * dk, DType::F32, "state", at);
    expect(g, n.output, BH * dv, act, "o", at);
}

void check_rmsnorm(const plan::Graph& g, const plan::Node& n, const RmsNormAttrs& a, const std::string& at) {
    if (n.inputs.size() != 2) invalid(at + ": takes [x, scale], got " + std::to_string(n.inputs.size()) + " inputs");
    if (a.rows < 0) invalid(at + ": rows must be >= 0");
    positive(a.dim, "dim", at);
    if (!(a.eps >= 0.f)) invalid(at + ": eps must be >= 0");
    if (a.dim > 1024) throw Error(RHZ_ERR_UNSUPPORTED, at + ": dim " + std::to_string(a.dim) + " exceeds 1024");
    const DType act = g.desc(n.inputs[0]).dtype;
    act_dtype(act, at);
    expect(g, n.inputs[0], std::size_t(a.rows) * a.dim, act, "x", at);
    expect(g, n.inputs[1], std::size_t(a.dim), DType::F32, "scale", at);
    expect(g, n.output, std::size_t(a.rows) * a.dim, act, "y", at);
}

}  // namespace

std::size_t CompiledPlan::offset(TensorId t) const {
    const plan::TensorDesc& d = graph_.desc(t);
    if (d.is_param) invalid("tensor " + std::to_string(t) + " '" + d.name + "' is a parameter: it has a binding, not an offset");
    const plan::Interval* i = arena_.find(t);
    if (!i) invalid("tensor " + std::to_string(t) + " '" + d.name + "' is used by no node and has no arena bytes");
    return i->offset;
}

CompiledPlan compile(const plan::Graph& graph, const std::map<std::size_t, NodeAttrs>& attrs) {
    graph.validate();
    CompiledPlan cp;
    cp.graph_ = graph;
    std::size_t cu_bytes = 0;
    for (std::size_t idx = 0; idx < graph.nodes().size(); ++idx) {
        const plan::Node& n = graph.nodes()[idx];
        const std::string at = where(idx, n);
        if (n.op != OpKind::DeltaScan && n.op != OpKind::DeltaStep && n.op != OpKind::RmsNorm)
            throw Error(RHZ_ERR_UNSUPPORTED, at + ": no MI355X kernel for this op");
        const auto it = attrs.find(idx);
        if (it == attrs.end()) invalid(at + ": no attributes given");
        CompiledPlan::Step step{idx, it->second, 0};
        if (n.op == OpKind::DeltaScan) {
            const auto* a = std::get_if<DeltaScanAttrs>(&it->second);
            if (!a) invalid(at + ": needs DeltaScanAttrs");
            cp.workspace_bytes_ = std::max(cp.workspace_bytes_, check_scan(graph, n, *a, at));
            if (!a->cu_seqlens.empty()) {
                step.cu_offset = cu_bytes;
                cu_bytes += align_up(a->cu_seqlens.size() * sizeof(int32_t));
            }
        } else if (n.op == OpKind::DeltaStep) {
            const auto* a = std::get_if<DeltaStepAttrs>(&it->second);
            if (!a) invalid(at + ": needs DeltaStepAttrs");
            check_step(graph, n, *a, at);
        } else {
            const auto* a = std::get_if<RmsNormAttrs>(&it->second);
            if (!a) invalid(at + ": needs RmsNormAttrs");
            check_rmsnorm(graph, n, *a, at);
        }
        cp.steps_.push_back(std::move(step));
    }
    for (const auto& [idx, a] : attrs)
        if (idx >= graph.nodes().size()) invalid("attributes given for node " + std::to_string(idx) + ", which does not exist");
    cp.arena_ = plan::plan(graph, /*pin_boundary=*/true);
    cp.cu_base_ = align_up(cp.arena_.total_bytes);
    cp.workspace_offset_ = cp.cu_base_ + cu_bytes;
    cp.device_bytes_ = cp.workspace_offset_ + align_up(cp.workspace_bytes_);
    return cp;
}

Executor::Executor(CompiledPlan plan) : plan_(std::move(plan)) {
    if (plan_.device_bytes_) {
        hip_check(hipMalloc(&base_, plan_.device_bytes_), "hipMalloc");
        try {
            hip_check(hipMemset(base_, 0, plan_.device_bytes_), "hipMemset");
            for (const auto& s : plan_.steps_)
                if (const auto* a = std::get_if<DeltaScanAttrs>(&s.attrs); a && !a->cu_seqlens.empty())
                    hip_check(hipMemcpy(static_cast<char*>(base_) + plan_.cu_base_ + s.cu_offset, a->cu_seqlens.data(),
                                        a->cu_seqlens.size() * sizeof(int32_t), hipMemcpyHostToDevice),
                              "hipMemcpy");
        } catch (...) {
            (void)hipFree(base_);
            throw;
        }
    }
}

Executor::~Executor() {
    release_graph();
    if (base_) (void)hipFree(base_);
}

void Executor::release_graph() {
    if (graph_exec_) (void)hipGraphExecDestroy(graph_exec_);
    if (graph_) (void)hipGraphDestroy(graph_);
    graph_exec_ = nullptr;
    graph_ = nullptr;
}

void Executor::bind(TensorId param, void* device_ptr) {
    const plan::TensorDesc& d = plan_.graph_.desc(param);
    if (!d.is_param) invalid("tensor " + std::to_string(param) + " '" + d.name + "' lives in the arena; only parameters are bound");
    bound_[param] = device_ptr;
}

void* Executor::data(TensorId t) const {
    if (plan_.graph_.desc(t).is_param) {
        const auto it = bound_.find(t);
        if (it == bound_.end() || !it->second)
            invalid("parameter " + std::to_string(t) + " '" + plan_.graph_.desc(t).name + "' is not bound");
        return it->second;
    }
    return static_cast<char*>(base_) + plan_.offset(t);
}

void Executor::run(hipStream_t stream) {
    // Resolve every address first, so an unbound parameter launches nothing.
    std::vector<std::vector<void*>> ptrs;
    for (const auto& s : plan_.steps_) {
        const plan::Node& n = plan_.graph_.nodes()[s.node];
        std::vector<void*> p;
        for (TensorId i : n.inputs) p.push_back(data(i));
        p.push_back(data(n.output));
        ptrs.push_back(std::move(p));
    }
    for (std::size_t si = 0; si < plan_.steps_.size(); ++si) {
        const auto& s = plan_.steps_[si];
        const plan::Node& n = plan_.graph_.nodes()[s.node];
        const std::vector<void*>& p = ptrs[si];
        const std::string at = where(s.node, n);
        if (const auto* a = std::get_if<DeltaScanAttrs>(&s.attrs)) {
            rhz_gdr_prefill_args pa{};
            pa.batch = a->batch;
            pa.seq_len = a->seq_len;
            pa.heads = a->heads;
            pa.d_k = a->d_k;
            pa.d_v = a->d_v;
            pa.chunk = a->chunk;
            pa.dtype = act_dtype(plan_.graph_.desc(n.inputs[0]).dtype, at);
            pa.gate_kind = a->gate_kind;
            pa.algo = a->algo;
            pa.q = p[0];
            pa.k = p[1];
            pa.v = p[2];
            pa.gate = static_cast<const float*>(p[3]);
            pa.beta = static_cast<const float*>(p[4]);
            if (!a->cu_seqlens.empty())
                pa.cu_seqlens = reinterpret_cast<const int32_t*>(static_cast<char*>(base_) + plan_.cu_base_ + s.cu_offset);
            if (n.inputs.size() == 6) {
                // initial and final state share the buffer: every thread reads its
                // slice of the state before it writes the same slice back.
                pa.initial_state = static_cast<const float*>(p[5]);
                pa.final_state = static_cast<float*>(p[5]);
            }
            pa.o = p.back();
            pa.workspace = plan_.workspace_bytes_ ? static_cast<char*>(base_) + plan_.workspace_offset_ : nullptr;
            pa.workspace_bytes = plan_.workspace_bytes_;
            check_status(rhz_gdr_prefill(&pa, stream), at);
        } else if (const auto* a = std::get_if<DeltaStepAttrs>(&s.attrs)) {
            rhz_gdr_decode_args da{};
            da.batch = a->batch;
            da.heads = a->heads;
            da.d_k = a->d_k;
            da.d_v = a->d_v;
            da.dtype = act_dtype(plan_.graph_.desc(n.inputs[0]).dtype, at);
            da.gate_kind = a->gate_kind;
            da.q = p[0];
            da.k = p[1];
            da.v = p[2];
            da.gate = static_cast<const float*>(p[3]);
            da.beta = static_cast<const float*>(p[4]);
            da.state = static_cast<float*>(p[5]);
            da.o = p.back();
            check_status(rhz_gdr_decode_step(&da, stream), at);
        } else {
            const auto& r = std::get<RmsNormAttrs>(s.attrs);
            rhz_rmsnorm_args ra{};
            ra.rows = r.rows;
            ra.dim = r.dim;
            ra.dtype = act_dtype(plan_.graph_.desc(n.inputs[0]).dtype, at);
            ra.eps = r.eps;
            ra.x = p[0];
            ra.scale = static_cast<const float*>(p[1]);
            ra.y = p.back();
            check_status(rhz_rmsnorm_heads(&ra, stream), at);
        }
    }
}

void Executor::capture(hipStream_t stream) {
    if (!stream) invalid("capture needs a non-default stream");
    release_graph();
    hip_check(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
    try {
        run(stream);
    } catch (...) {
        hipGraph_t g = nullptr;
        (void)hipStreamEndCapture(stream, &g);
        if (g) (void)hipGraphDestroy(g);
        throw;
    }
    hip_check(hipStreamEndCapture(stream, &graph_), "hipStreamEndCapture");
    hip_check(hipGraphInstantiate(&graph_exec_, graph_, nullptr, nullptr, 0), "hipGraphInstantiate");
}

void Executor::replay(hipStream_t stream) {
    if (!graph_exec_) invalid("replay before capture");
    hip_check(hipGraphLaunch(graph_exec_, stream), "hipGraphLaunch");
}

}  // namespace exec
}  // namespace rhizome
