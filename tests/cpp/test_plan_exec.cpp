// Tests of the C++ plan layer (rhizome_amd/host/rhizome_plan.hpp) and of the
// executor over it (rhizome_exec.hpp).
//
//   test_plan_exec            every test (needs a GPU)
//   test_plan_exec --cpu      the tests that make no GPU call: the
//                             reference's own graph and arena unit tests
//                             (graph.rs and arena.rs tests, dtype.rs:158-162),
//                             a hand-computed plan, and the executor's
//                             plan-time errors
//   test_plan_exec --dump N   print N seeded random graphs with their plans
//                             (reference liveness and the executor's), for
//                             the pure-Python planner oracle to compare
//
// The GPU tests run graphs of DeltaScan / DeltaStep / RmsNorm nodes through
// the executor and compare every output with the f64 oracle
// (oracle/gdr_oracle.c) on the same inputs, and replay a captured HIP graph
// against the eager run bit for bit.
//
// Exit status 0 when every test passes.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

#include "rhizome_exec.hpp"
#include "rhizome_plan.hpp"

using namespace rhizome;
using plan::DType;
using plan::OpKind;
using plan::TensorId;

// The f64 oracle (oracle/gdr_oracle.c), test infrastructure only.
extern "C" {
void orc_philox_normal(uint64_t seed, uint64_t stream, int64_t n, double mean, double std_, double* out,
                       int nthreads);
void orc_l2norm_rows(double* x, int64_t rows, int64_t d, double scale, int nthreads);
void orc_sigmoid_vec(const double* z, int64_t n, double* out);
void orc_neg_softplus_vec(const double* z, int64_t n, double* out);
void orc_exp_vec(const double* z, int64_t n, double* out);
void orc_rmsnorm_rows(int64_t rows, int64_t dim, const double* x, const double* scale, double eps, double* y);
void orc_gdr_prefill_batched(int64_t n_seqs, const int64_t* cu_seqlens, int64_t heads, int64_t dk, int64_t dv,
                             const double* q, const double* k, const double* v, const double* alpha,
                             const double* beta, const double* init, double* o, double* final_state,
                             int nthreads);
void orc_gdr_decode_batched(int64_t batch, int64_t heads, int64_t dk, int64_t dv, const double* q,
                            const double* k, const double* v, const double* alpha, const double* beta,
                            double* state, double* o, int nthreads);
}

namespace {

int g_failed = 0;

#define EXPECT(cond)                                                              \
    do {                                                                          \
        if (!(cond)) throw std::runtime_error(std::string("expected: ") + #cond); \
    } while (0)

void run(const char* name, const std::function<void()>& fn) {
    try {
        fn();
        std::printf("PASS %s\n", name);
    } catch (const std::exception& e) {
        ++g_failed;
        std::printf("FAIL %s: %s\n", name, e.what());
    }
    std::fflush(stdout);
}

// fn must throw rhizome::Error with this status.
void expect_error(int32_t status, const std::function<void()>& fn, const char* what) {
    try {
        fn();
    } catch (const Error& e) {
        if (e.status() != status)
            throw std::runtime_error(std::string(what) + ": status " + std::to_string(e.status()) + " (" + e.what() +
                                     "), expected " + std::to_string(status));
        std::printf("  %s -> %s\n", what, e.what());
        return;
    }
    throw std::runtime_error(std::string(what) + ": no error thrown");
}

// ------------------------------------------------------------ reference tests
plan::Graph chain(std::size_t len) {  // arena.rs:151-160
    plan::Graph g;
    TensorId cur = g.tensor("x", 1024, DType::F32, false);
    for (std::size_t i = 0; i < len; ++i) cur = g.push(OpKind::Silu, {cur}, "h" + std::to_string(i), 1024, DType::F32);
    return g;
}

plan::Graph mlp_graph() {  // graph.rs tests: mlp_graph
    plan::Graph g;
    const TensorId x = g.tensor("x", 16, DType::F32, false);
    const TensorId w1 = g.tensor("w1", 16 * 32, DType::BF16, true);
    const TensorId w2 = g.tensor("w2", 32 * 16, DType::BF16, true);
    const TensorId h = g.push(OpKind::Linear, {x, w1}, "h", 32, DType::F32);
    const TensorId a = g.push(OpKind::Silu, {h}, "a", 32, DType::F32);
    g.push(OpKind::Linear, {a, w2}, "y", 16, DType::F32);
    return g;
}

void dtype_bytes() {  // dtype.rs:158-162, plus the MX scale bytes
    EXPECT(plan::block_size(DType::MXFP4) == 32);
    EXPECT(plan::bytes_for(DType::BF16, 10) == 20);
    EXPECT(plan::bytes_for(DType::MXFP4, 64) == 32 + 2);
    EXPECT(plan::bytes_for(DType::MXINT4, 33) == 17 + 2);
    EXPECT(plan::bytes_for(DType::F32, 3) == 12);
    EXPECT(plan::bytes_for(DType::F8E4M3, 5) == 5);
}

void op_names() {  // graph.rs tests: op_metadata_is_consistent, and the GDR names (graph.rs:124-125)
    EXPECT(std::string(plan::name(OpKind::MlaDecode)) == "mla_decode");
    EXPECT(std::string(plan::name(OpKind::DeltaScan)) == "gated_delta_scan_chunked");
    EXPECT(std::string(plan::name(OpKind::DeltaStep)) == "gated_delta_step");
    EXPECT(std::string(plan::name(OpKind::RmsNorm)) == "rmsnorm");
    EXPECT(std::string(plan::name(OpKind::Sample)) == "sampling");
}

void valid_graph_passes_validation() { mlp_graph().validate(); }

void unknown_input_is_rejected() {
    plan::Graph g;
    expect_error(RHZ_ERR_INVALID_ARG, [&] { g.push(OpKind::Silu, {7}, "y", 4, DType::F32); }, "push with unknown input");
}

void chain_reuses_memory() {  // arena.rs:162-167
    const plan::ArenaPlan p = plan::plan(chain(8));
    EXPECT(p.total_bytes < p.unplanned_bytes());
    p.verify();
}

void offsets_are_aligned() {  // arena.rs:169-175
    const plan::ArenaPlan p = plan::plan(chain(5));
    for (const auto& i : p.intervals) EXPECT(i.offset % plan::kAlign == 0);
}

void parameters_are_not_placed_in_the_arena() {  // arena.rs:177-186
    plan::Graph g;
    const TensorId x = g.tensor("x", 16, DType::F32, false);
    const TensorId w = g.tensor("w", 4096, DType::BF16, true);
    g.push(OpKind::Linear, {x, w}, "y", 16, DType::F32);
    const plan::ArenaPlan p = plan::plan(g);
    for (const auto& i : p.intervals) EXPECT(i.tensor != w);
}

void long_lived_tensor_does_not_alias() {  // arena.rs:188-215
    plan::Graph g;
    const TensorId x = g.tensor("x", 256, DType::F32, false);
    const TensorId a = g.push(OpKind::Silu, {x}, "a", 256, DType::F32);
    const TensorId b = g.push(OpKind::Silu, {a}, "b", 256, DType::F32);
    g.push(OpKind::Add, {x, b}, "c", 256, DType::F32);
    const plan::ArenaPlan p = plan::plan(g);
    p.verify();
    EXPECT(!p.find(x)->overlaps_memory(*p.find(b)));
}

void detects_injected_conflicts() {  // arena.rs:217-227
    plan::ArenaPlan p = plan::plan(chain(3));
    const plan::Interval first = p.intervals[0];
    for (auto& i : p.intervals) {
        i.offset = first.offset;
        i.start = 0;
        i.end = 10;
    }
    expect_error(RHZ_ERR_INVALID_ARG, [&] { p.verify(); }, "verify of an injected conflict");
}

// Worked by hand: x [0,0], h0 [0,1], h1 [1,2], h2 [2,2], all 4096 B, placed
// in id order: x at 0; h0 meets x -> 4096; h1 meets h0 only -> 0 fits below
// it; h2 meets h1 only -> 4096.
void chain3_hand_computed() {
    const plan::ArenaPlan p = plan::plan(chain(3));
    EXPECT(p.intervals.size() == 4);
    const std::size_t off[4] = {0, 4096, 0, 4096}, st[4] = {0, 0, 1, 2}, en[4] = {0, 1, 2, 2};
    for (std::size_t i = 0; i < 4; ++i) {
        EXPECT(p.intervals[i].tensor == i);
        EXPECT(p.intervals[i].offset == off[i] && p.intervals[i].size == 4096);
        EXPECT(p.intervals[i].start == st[i] && p.intervals[i].end == en[i]);
    }
    EXPECT(p.total_bytes == 8192 && p.unplanned_bytes() == 16384);
}

// A graph input first read by a late node: the reference's liveness lets it
// share bytes with an intermediate written earlier (so a value written before
// the run would be overwritten by node 0); the executor's liveness keeps
// every input and output apart from everything.
void boundary_tensors_are_pinned() {
    plan::Graph g;
    const TensorId x = g.tensor("x", 1024, DType::F32, false);
    const TensorId h0 = g.push(OpKind::Silu, {x}, "h0", 1024, DType::F32);
    const TensorId h1 = g.push(OpKind::Silu, {h0}, "h1", 1024, DType::F32);
    const TensorId late = g.tensor("late", 1024, DType::F32, false);
    const TensorId z = g.push(OpKind::Add, {h1, late}, "z", 1024, DType::F32);
    const plan::ArenaPlan ref = plan::plan(g);
    EXPECT(ref.find(late)->offset == ref.find(h0)->offset);  // the hazard, as the reference plans it
    const plan::ArenaPlan pin = plan::plan(g, true);
    pin.verify();
    for (TensorId t : {x, late, z}) {
        EXPECT(pin.find(t)->start == 0 && pin.find(t)->end == 2);
        for (const auto& o : pin.intervals)
            if (o.tensor != t) EXPECT(!pin.find(t)->overlaps_memory(o));
    }
    EXPECT(pin.find(h0)->start == 0 && pin.find(h0)->end == 1 && pin.find(h1)->start == 1);
}

// ------------------------------------------------------------ executor: plan time
struct ScanGraph {
    plan::Graph g;
    TensorId q, k, v, gate, beta, state, o;
    std::map<std::size_t, exec::NodeAttrs> attrs;
};

// One DeltaScan over a packed batch; state optional (as a parameter or in the arena).
ScanGraph scan_graph(const std::vector<int32_t>& cu, int32_t H, int32_t dk, int32_t dv, DType act, int state_kind,
                     int32_t algo = RHZ_ALGO_AUTO) {
    ScanGraph s;
    const std::size_t tok = cu.back(), N = cu.size() - 1;
    s.q = s.g.tensor("q", tok * H * dk, act, false);
    s.k = s.g.tensor("k", tok * H * dk, act, false);
    s.v = s.g.tensor("v", tok * H * dv, act, false);
    s.gate = s.g.tensor("gate", tok * H, DType::F32, false);
    s.beta = s.g.tensor("beta", tok * H, DType::F32, false);
    std::vector<TensorId> ins{s.q, s.k, s.v, s.gate, s.beta};
    s.state = 0;
    if (state_kind) {
        s.state = s.g.tensor("state", N * H * dv * dk, DType::F32, state_kind == 1);
        ins.push_back(s.state);
    }
    s.o = s.g.push(OpKind::DeltaScan, ins, "o", tok * H * dv, act);
    exec::DeltaScanAttrs a;
    a.batch = int32_t(N);
    a.seq_len = int32_t(tok);
    a.heads = H;
    a.d_k = dk;
    a.d_v = dv;
    a.algo = algo;
    a.cu_seqlens = cu;
    s.attrs[0] = a;
    return s;
}

void compile_layout() {
    ScanGraph s = scan_graph({0, 70, 70, 200}, 2, 64, 64, DType::BF16, 1);
    const exec::CompiledPlan cp = exec::compile(s.g, s.attrs);
    EXPECT(cp.workspace_bytes() == 256);  // the sequence order of 3 sequences, rounded to 256 B
    EXPECT(cp.arena().find(s.state) == nullptr);
    std::size_t end = 0;
    for (const auto& i : cp.arena().intervals) {
        EXPECT(i.offset % 256 == 0);
        EXPECT(i.start == 0 && i.end == 0);
        end = std::max(end, i.offset + i.size);
    }
    EXPECT(end == cp.arena().total_bytes);
    // arena, then the 4 packed offsets (256 B), then the workspace (256 B)
    EXPECT(cp.device_bytes() == (cp.arena().total_bytes + 255) / 256 * 256 + 256 + 256);
    EXPECT(cp.offset(s.q) == cp.arena().find(s.q)->offset);
    expect_error(RHZ_ERR_INVALID_ARG, [&] { cp.offset(s.state); }, "offset of a parameter");
}

void compile_errors() {
    {   // an op the library has no kernel for
        plan::Graph g;
        const TensorId x = g.tensor("x", 16, DType::F32, false);
        g.push(OpKind::Silu, {x}, "y", 16, DType::F32);
        expect_error(RHZ_ERR_UNSUPPORTED, [&] { exec::compile(g, {}); }, "silu node");
    }
    {   // no attributes for the node
        ScanGraph s = scan_graph({0, 10}, 1, 32, 32, DType::BF16, 0);
        expect_error(RHZ_ERR_INVALID_ARG, [&] { exec::compile(s.g, {}); }, "missing attributes");
        expect_error(RHZ_ERR_INVALID_ARG, [&] { exec::compile(s.g, {{0, exec::DeltaStepAttrs{}}}); },
                     "attributes of another op");
        auto extra = s.attrs;
        extra[5] = exec::RmsNormAttrs{};
        expect_error(RHZ_ERR_INVALID_ARG, [&] { exec::compile(s.g, extra); }, "attributes for a missing node");
    }
    {   // shapes that disagree with the attributes
        ScanGraph s = scan_graph({0, 10}, 1, 32, 32, DType::BF16, 0);
        std::get<exec::DeltaScanAttrs>(s.attrs[0]).heads = 2;
        expect_error(RHZ_ERR_INVALID_ARG, [&] { exec::compile(s.g, s.attrs); }, "heads disagree with q");
        ScanGraph t = scan_graph({0, 10}, 1, 32, 32, DType::BF16, 0);
        std::get<exec::DeltaScanAttrs>(t.attrs[0]).cu_seqlens = {0, 11};
        expect_error(RHZ_ERR_INVALID_ARG, [&] { exec::compile(t.g, t.attrs); }, "cu_seqlens past seq_len");
        std::get<exec::DeltaScanAttrs>(t.attrs[0]).cu_seqlens = {0, 6, 4, 10};
        std::get<exec::DeltaScanAttrs>(t.attrs[0]).batch = 3;
        expect_error(RHZ_ERR_INVALID_ARG, [&] { exec::compile(t.g, t.attrs); }, "decreasing cu_seqlens");
    }
    {   // formats and sizes the library does not run
        ScanGraph s = scan_graph({0, 10}, 1, 32, 32, DType::F32, 0, RHZ_ALGO_CHUNKED);
        expect_error(RHZ_ERR_UNSUPPORTED, [&] { exec::compile(s.g, s.attrs); }, "CHUNKED with f32");
        ScanGraph t = scan_graph({0, 10}, 1, 300, 32, DType::BF16, 0);
        expect_error(RHZ_ERR_UNSUPPORTED, [&] { exec::compile(t.g, t.attrs); }, "d_k = 300");
        ScanGraph u = scan_graph({0, 10}, 1, 32, 32, DType::F8E4M3, 0);
        expect_error(RHZ_ERR_UNSUPPORTED, [&] { exec::compile(u.g, u.attrs); }, "f8 activations");
    }
    {   // DeltaStep without a state operand, and with a state of the wrong size
        auto step_graph = [](bool with_state) {
            plan::Graph g;
            std::vector<TensorId> ins{g.tensor("q", 64, DType::F32, false), g.tensor("k", 64, DType::F32, false),
                                      g.tensor("v", 64, DType::F32, false), g.tensor("a", 2, DType::F32, false),
                                      g.tensor("b", 2, DType::F32, false)};
            if (with_state) ins.push_back(g.tensor("s", 2 * 32 * 31, DType::F32, true));
            g.push(OpKind::DeltaStep, ins, "o", 64, DType::F32);
            return g;
        };
        const exec::DeltaStepAttrs at{1, 2, 32, 32};
        expect_error(RHZ_ERR_INVALID_ARG, [&] { exec::compile(step_graph(false), {{0, at}}); }, "step with 5 inputs");
        expect_error(RHZ_ERR_INVALID_ARG, [&] { exec::compile(step_graph(true), {{0, at}}); }, "state of the wrong size");
    }
    {   // RmsNorm: dim over the supported 1024
        plan::Graph g;
        const TensorId x = g.tensor("x", 2 * 2048, DType::BF16, false), w = g.tensor("w", 2048, DType::F32, true);
        g.push(OpKind::RmsNorm, {x, w}, "y", 2 * 2048, DType::BF16);
        expect_error(RHZ_ERR_UNSUPPORTED, [&] { exec::compile(g, {{0, exec::RmsNormAttrs{2, 2048, 1e-6f}}}); },
                     "rmsnorm dim 2048");
    }
}

// ------------------------------------------------------------ random graphs for the planner oracle
struct Rng {
    uint64_t s;
    uint64_t next() {  // splitmix64
        uint64_t z = (s += 0x9E3779B97F4A7C15ull);
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    }
    std::size_t below(std::size_t n) { return next() % n; }
};

void dump_graphs(int count) {
    Rng r{12345};
    const DType dts[] = {DType::F64, DType::F32, DType::BF16, DType::F8E4M3, DType::MXFP4, DType::MXINT4, DType::I8};
    // A few sizes recur so that ties in the largest-first order are exercised.
    const std::size_t common[] = {64, 256, 1000, 1024, 4096};
    for (int gi = 0; gi < count; ++gi) {
        plan::Graph g;
        const std::size_t n_in = 1 + r.below(4), n_nodes = r.below(14);
        auto elems = [&] { return r.below(3) ? common[r.below(5)] : 1 + r.below(6000); };
        for (std::size_t i = 0; i < n_in; ++i)
            g.tensor("t" + std::to_string(i), elems(), dts[r.below(7)], r.below(4) == 0);
        for (std::size_t nidx = 0; nidx < n_nodes; ++nidx) {
            // Late graph inputs as well as node outputs.
            if (r.below(5) == 0) g.tensor("in" + std::to_string(nidx), elems(), dts[r.below(7)], r.below(3) == 0);
            std::vector<TensorId> ins;
            const std::size_t k = 1 + r.below(3);
            for (std::size_t j = 0; j < k; ++j) ins.push_back(r.below(g.tensors().size()));
            g.push(static_cast<OpKind>(r.below(23)), ins, "n" + std::to_string(nidx), elems(), dts[r.below(7)]);
        }
        std::printf("graph %d\n", gi);
        for (const auto& t : g.tensors())
            std::printf("t %zu %s %d\n", t.elems, plan::dtype_name(t.dtype), t.is_param ? 1 : 0);
        for (const auto& n : g.nodes()) {
            std::printf("n %d %zu", static_cast<int>(n.op), n.output);
            for (TensorId i : n.inputs) std::printf(" %zu", i);
            std::printf("\n");
        }
        for (int pin = 0; pin < 2; ++pin) {
            const plan::ArenaPlan p = plan::plan(g, pin == 1);
            std::printf("plan %d %zu\n", pin, p.total_bytes);
            for (const auto& i : p.intervals)
                std::printf("i %zu %zu %zu %zu %zu\n", i.tensor, i.start, i.end, i.offset, i.size);
        }
    }
}

// ------------------------------------------------------------ executor on the GPU
void hip_ok(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

uint16_t to_bf16(float f) {  // round to nearest even (inputs are finite)
    uint32_t u;
    std::memcpy(&u, &f, 4);
    u += 0x7fffu + ((u >> 16) & 1u);
    return uint16_t(u >> 16);
}

float from_bf16(uint16_t h) {
    const uint32_t u = uint32_t(h) << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

// Copy f64 values to the device as `dt`; returns the values the device holds.
std::vector<double> put(void* dst, const std::vector<double>& x, DType dt) {
    std::vector<double> held(x.size());
    if (dt == DType::BF16) {
        std::vector<uint16_t> h(x.size());
        for (std::size_t i = 0; i < x.size(); ++i) {
            h[i] = to_bf16(float(x[i]));
            held[i] = from_bf16(h[i]);
        }
        hip_ok(hipMemcpy(dst, h.data(), h.size() * 2, hipMemcpyHostToDevice), "hipMemcpy");
    } else {
        std::vector<float> h(x.begin(), x.end());
        for (std::size_t i = 0; i < x.size(); ++i) held[i] = h[i];
        hip_ok(hipMemcpy(dst, h.data(), h.size() * 4, hipMemcpyHostToDevice), "hipMemcpy");
    }
    return held;
}

std::vector<double> get(const void* src, std::size_t n, DType dt) {
    std::vector<double> out(n);
    if (dt == DType::BF16) {
        std::vector<uint16_t> h(n);
        hip_ok(hipMemcpy(h.data(), src, n * 2, hipMemcpyDeviceToHost), "hipMemcpy");
        for (std::size_t i = 0; i < n; ++i) out[i] = from_bf16(h[i]);
    } else {
        std::vector<float> h(n);
        hip_ok(hipMemcpy(h.data(), src, n * 4, hipMemcpyDeviceToHost), "hipMemcpy");
        for (std::size_t i = 0; i < n; ++i) out[i] = h[i];
    }
    return out;
}

std::vector<uint8_t> raw(const void* src, std::size_t bytes) {
    std::vector<uint8_t> h(bytes);
    hip_ok(hipMemcpy(h.data(), src, bytes, hipMemcpyDeviceToHost), "hipMemcpy");
    return h;
}

// |x - y| <= atol_rms * RMS(y) + rtol * |y| elementwise, as the Python parity tests.
void check_close(const std::vector<double>& x, const std::vector<double>& y, double rtol, double atol_rms,
                 const char* what) {
    EXPECT(x.size() == y.size());
    double ss = 0.0;
    for (double v : y) ss += v * v;
    const double atol = y.empty() ? 0.0 : atol_rms * std::sqrt(ss / y.size());
    double worst = 0.0;
    for (std::size_t i = 0; i < x.size(); ++i) {
        if (!std::isfinite(x[i])) throw std::runtime_error(std::string(what) + ": non-finite output");
        const double ratio = std::fabs(x[i] - y[i]) / std::max(atol + rtol * std::fabs(y[i]), 1e-300);
        worst = std::max(worst, ratio);
        if (ratio > 1.0)
            throw std::runtime_error(std::string(what) + ": element " + std::to_string(i) + " " + std::to_string(x[i]) +
                                     " vs " + std::to_string(y[i]));
    }
    std::printf("  %s: max err/bound %.3f\n", what, worst);
}

std::vector<double> normal(uint64_t seed, uint64_t stream, std::size_t n, double mean = 0.0, double sd = 1.0) {
    std::vector<double> x(n);
    orc_philox_normal(seed, stream, int64_t(n), mean, sd, x.data(), 1);
    return x;
}

std::vector<double> unit_rows(uint64_t seed, uint64_t stream, std::size_t rows, std::size_t d) {
    std::vector<double> x = normal(seed, stream, rows * d);
    orc_l2norm_rows(x.data(), int64_t(rows), int64_t(d), 1.0, 1);
    return x;
}

std::vector<double> map(std::vector<double> x, void (*f)(const double*, int64_t, double*)) {
    f(x.data(), int64_t(x.size()), x.data());
    return x;
}

// Inputs of one GDR call over `rows` (token, head) rows, as the f64 values
// the oracle sees after rounding to the device formats.
struct Gdr {
    std::vector<double> q, k, v, g, beta;
};

Gdr fill_gdr(exec::Executor& ex, TensorId q, TensorId k, TensorId v, TensorId g, TensorId b, std::size_t rows,
             std::size_t dk, std::size_t dv, DType act, uint64_t seed) {
    Gdr in;
    in.q = put(ex.data(q), unit_rows(seed, 1, rows, dk), act);
    in.k = put(ex.data(k), unit_rows(seed, 2, rows, dk), act);
    in.v = put(ex.data(v), normal(seed, 3, rows * dv), act);
    in.beta = put(ex.data(b), map(normal(seed, 4, rows), orc_sigmoid_vec), DType::F32);
    in.g = put(ex.data(g), map(normal(seed, 5, rows), orc_neg_softplus_vec), DType::F32);
    return in;
}

// Device buffer owned by a test (parameters and caches bound to the executor).
struct Dev {
    void* p = nullptr;
    explicit Dev(std::size_t bytes) { hip_ok(hipMalloc(&p, bytes), "hipMalloc"); }
    ~Dev() { (void)hipFree(p); }
};

// bf16 chunked prefill over a packed batch with an empty sequence; the
// state is a parameter bound by the caller, read and overwritten in place.
void exec_scan_packed_state() {
    const std::vector<int32_t> cu{0, 70, 70, 200};
    const std::size_t H = 2, dk = 64, dv = 64, N = 3, tok = 200;
    ScanGraph s = scan_graph(cu, H, dk, dv, DType::BF16, 1);
    exec::Executor ex(exec::compile(s.g, s.attrs));
    Dev state(N * H * dv * dk * 4);
    ex.bind(s.state, state.p);
    const Gdr in = fill_gdr(ex, s.q, s.k, s.v, s.gate, s.beta, tok * H, dk, dv, DType::BF16, 11);
    std::vector<double> st = put(state.p, normal(11, 6, N * H * dv * dk, 0.0, 0.02), DType::F32);
    ex.run();
    hip_ok(hipDeviceSynchronize(), "sync");
    const std::vector<int64_t> cu64(cu.begin(), cu.end());
    std::vector<double> o(tok * H * dv), fin(st.size());
    orc_gdr_prefill_batched(N, cu64.data(), H, dk, dv, in.q.data(), in.k.data(), in.v.data(),
                            map(in.g, orc_exp_vec).data(), in.beta.data(), st.data(), o.data(), fin.data(), 8);
    check_close(get(ex.data(s.o), o.size(), DType::BF16), o, 2e-2, 1e-2, "o");
    check_close(get(state.p, fin.size(), DType::F32), fin, 2e-2, 1e-2, "state (in place)");
}

// RmsNorm -> DeltaScan -> RmsNorm -> DeltaStep in f32 on a dense batch, the
// state living in the arena (a graph input: written before the run, read
// after it).  Each output against the oracle's composition of the same steps.
void exec_chain_f32() {
    const std::size_t B = 2, T = 50, H = 2, dk = 32, dv = 48, rows = B * T * H;
    plan::Graph g;
    const TensorId xq = g.tensor("xq", rows * dk, DType::F32, false);
    const TensorId wq = g.tensor("wq", dk, DType::F32, true);
    const TensorId k = g.tensor("k", rows * dk, DType::F32, false);
    const TensorId v = g.tensor("v", rows * dv, DType::F32, false);
    const TensorId gt = g.tensor("g", B * T * H, DType::F32, false);
    const TensorId bt = g.tensor("beta", B * T * H, DType::F32, false);
    const TensorId st = g.tensor("state", B * H * dv * dk, DType::F32, false);
    const TensorId q = g.push(OpKind::RmsNorm, {xq, wq}, "q", rows * dk, DType::F32);
    const TensorId o = g.push(OpKind::DeltaScan, {q, k, v, gt, bt, st}, "o", rows * dv, DType::F32);
    const TensorId wo = g.tensor("wo", dv, DType::F32, true);
    const TensorId y = g.push(OpKind::RmsNorm, {o, wo}, "y", rows * dv, DType::F32);
    const TensorId q1 = g.tensor("q1", B * H * dk, DType::F32, false), k1 = g.tensor("k1", B * H * dk, DType::F32, false);
    const TensorId v1 = g.tensor("v1", B * H * dv, DType::F32, false), g1 = g.tensor("g1", B * H, DType::F32, false);
    const TensorId b1 = g.tensor("b1", B * H, DType::F32, false);
    const TensorId o1 = g.push(OpKind::DeltaStep, {q1, k1, v1, g1, b1, st}, "o1", B * H * dv, DType::F32);
    exec::DeltaScanAttrs sa;
    sa.batch = B;
    sa.seq_len = T;
    sa.heads = H;
    sa.d_k = dk;
    sa.d_v = dv;
    const float eps = 1e-6f;
    std::map<std::size_t, exec::NodeAttrs> attrs{{0, exec::RmsNormAttrs{int32_t(rows), int32_t(dk), eps}},
                                                 {1, sa},
                                                 {2, exec::RmsNormAttrs{int32_t(rows), int32_t(dv), eps}},
                                                 {3, exec::DeltaStepAttrs{int32_t(B), int32_t(H), int32_t(dk), int32_t(dv)}}};
    const exec::CompiledPlan cp = exec::compile(g, attrs);
    // Intermediates keep their own live ranges; inputs and outputs span the run.
    EXPECT(cp.arena().find(q)->start == 0 && cp.arena().find(q)->end == 1);
    EXPECT(cp.arena().find(o)->start == 1 && cp.arena().find(o)->end == 2);
    EXPECT(cp.arena().find(st)->start == 0 && cp.arena().find(st)->end == 3);
    EXPECT(cp.arena().find(y)->end == 3 && cp.arena().find(q1)->start == 0);
    exec::Executor ex(cp);
    Dev wq_d(dk * 4), wo_d(dv * 4);
    ex.bind(wq, wq_d.p);
    ex.bind(wo, wo_d.p);
    const std::vector<double> xq_h = put(ex.data(xq), normal(21, 1, rows * dk, 0.0, 0.3), DType::F32);
    const std::vector<double> wq_h = put(wq_d.p, normal(21, 7, dk, 0.0, 1.0 / std::sqrt(double(dk))), DType::F32);
    const std::vector<double> wo_h = put(wo_d.p, normal(21, 8, dv), DType::F32);
    const std::vector<double> k_h = put(ex.data(k), unit_rows(21, 2, rows, dk), DType::F32);
    const std::vector<double> v_h = put(ex.data(v), normal(21, 3, rows * dv), DType::F32);
    const std::vector<double> b_h = put(ex.data(bt), map(normal(21, 4, B * T * H), orc_sigmoid_vec), DType::F32);
    const std::vector<double> g_h = put(ex.data(gt), map(normal(21, 5, B * T * H), orc_neg_softplus_vec), DType::F32);
    std::vector<double> s_h = put(ex.data(st), normal(21, 6, B * H * dv * dk, 0.0, 0.02), DType::F32);
    const Gdr d1 = fill_gdr(ex, q1, k1, v1, g1, b1, B * H, dk, dv, DType::F32, 22);
    ex.run();
    hip_ok(hipDeviceSynchronize(), "sync");

    std::vector<double> q_r(rows * dk), o_r(rows * dv), y_r(rows * dv), o1_r(B * H * dv);
    orc_rmsnorm_rows(rows, dk, xq_h.data(), wq_h.data(), eps, q_r.data());
    std::vector<int64_t> cu(B + 1);
    for (std::size_t b = 0; b <= B; ++b) cu[b] = int64_t(b * T);
    orc_gdr_prefill_batched(B, cu.data(), H, dk, dv, q_r.data(), k_h.data(), v_h.data(), map(g_h, orc_exp_vec).data(),
                            b_h.data(), s_h.data(), o_r.data(), s_h.data(), 8);
    orc_rmsnorm_rows(rows, dv, o_r.data(), wo_h.data(), eps, y_r.data());
    orc_gdr_decode_batched(B, H, dk, dv, d1.q.data(), d1.k.data(), d1.v.data(), map(d1.g, orc_exp_vec).data(),
                           d1.beta.data(), s_h.data(), o1_r.data(), 1);
    check_close(get(ex.data(q), q_r.size(), DType::F32), q_r, 1e-4, 1e-4, "q = rmsnorm(xq)");
    check_close(get(ex.data(y), y_r.size(), DType::F32), y_r, 1e-4, 1e-4, "y = rmsnorm(scan)");
    check_close(get(ex.data(o1), o1_r.size(), DType::F32), o1_r, 1e-4, 1e-4, "o1 = step");
    check_close(get(ex.data(st), s_h.size(), DType::F32), s_h, 1e-4, 1e-4, "state after scan and step");
}

// A captured run replayed three times, with eager runs in between, equals
// the eager run bit for bit (state reset to the same value before each).
void exec_capture_replay() {
    const std::vector<int32_t> cu{0, 100, 164, 300};
    const std::size_t H = 4, dk = 128, dv = 128, N = 3, tok = 300;
    ScanGraph s = scan_graph(cu, H, dk, dv, DType::BF16, 1);
    const TensorId w = s.g.tensor("w", dv, DType::F32, true);
    const TensorId y = s.g.push(OpKind::RmsNorm, {s.o, w}, "y", tok * H * dv, DType::BF16);
    s.attrs[1] = exec::RmsNormAttrs{int32_t(tok * H), int32_t(dv), 1e-6f};
    exec::Executor ex(exec::compile(s.g, s.attrs));
    const std::size_t sbytes = N * H * dv * dk * 4, ybytes = tok * H * dv * 2;
    Dev state(sbytes), state0(sbytes), wd(dv * 4);
    ex.bind(s.state, state.p);
    ex.bind(w, wd.p);
    fill_gdr(ex, s.q, s.k, s.v, s.gate, s.beta, tok * H, dk, dv, DType::BF16, 31);
    put(state0.p, normal(31, 6, N * H * dv * dk, 0.0, 0.02), DType::F32);
    put(wd.p, normal(31, 8, dv), DType::F32);
    hipStream_t stream;
    hip_ok(hipStreamCreate(&stream), "hipStreamCreate");
    auto reset = [&] { hip_ok(hipMemcpy(state.p, state0.p, sbytes, hipMemcpyDeviceToDevice), "reset"); };
    reset();
    ex.run(stream);
    hip_ok(hipStreamSynchronize(stream), "sync");
    const std::vector<uint8_t> y_eager = raw(ex.data(y), ybytes), s_eager = raw(state.p, sbytes);
    ex.capture(stream);
    for (int rep = 0; rep < 3; ++rep) {
        reset();
        hip_ok(hipMemset(ex.data(y), 0xff, ybytes), "poison y");
        ex.replay(stream);
        hip_ok(hipStreamSynchronize(stream), "sync");
        EXPECT(raw(ex.data(y), ybytes) == y_eager);
        EXPECT(raw(state.p, sbytes) == s_eager);
        reset();
        ex.run(stream);  // eager work between replays
        hip_ok(hipStreamSynchronize(stream), "sync");
        EXPECT(raw(ex.data(y), ybytes) == y_eager);
    }
    hip_ok(hipStreamDestroy(stream), "hipStreamDestroy");
}

void exec_unbound_parameter_launches_nothing() {
    ScanGraph s = scan_graph({0, 64}, 1, 32, 32, DType::BF16, 1);
    exec::Executor ex(exec::compile(s.g, s.attrs));
    hip_ok(hipMemset(ex.data(s.o), 0x5a, 64 * 32 * 2), "memset");
    expect_error(RHZ_ERR_INVALID_ARG, [&] { ex.run(); }, "run with the state unbound");
    hip_ok(hipDeviceSynchronize(), "sync");
    const std::vector<uint8_t> o = raw(ex.data(s.o), 64 * 32 * 2);
    for (uint8_t b : o) EXPECT(b == 0x5a);
    expect_error(RHZ_ERR_INVALID_ARG, [&] { ex.bind(s.q, nullptr); }, "binding an arena tensor");
}

}  // namespace

int main(int argc, char** argv) {
    if (argc > 2 && std::strcmp(argv[1], "--dump") == 0) {
        dump_graphs(std::atoi(argv[2]));
        return 0;
    }
    const bool cpu_only = argc > 1 && std::strcmp(argv[1], "--cpu") == 0;
    run("dtype_bytes", dtype_bytes);
    run("op_names", op_names);
    run("valid_graph_passes_validation", valid_graph_passes_validation);
    run("unknown_input_is_rejected", unknown_input_is_rejected);
    run("chain_reuses_memory", chain_reuses_memory);
    run("offsets_are_aligned", offsets_are_aligned);
    run("parameters_are_not_placed_in_the_arena", parameters_are_not_placed_in_the_arena);
    run("long_lived_tensor_does_not_alias", long_lived_tensor_does_not_alias);
    run("detects_injected_conflicts", detects_injected_conflicts);
    run("chain3_hand_computed", chain3_hand_computed);
    run("boundary_tensors_are_pinned", boundary_tensors_are_pinned);
    run("compile_layout", compile_layout);
    run("compile_errors", compile_errors);
    if (!cpu_only) {
        run("exec_scan_packed_state", exec_scan_packed_state);
        run("exec_chain_f32", exec_chain_f32);
        run("exec_capture_replay", exec_capture_replay);
        run("exec_unbound_parameter_launches_nothing", exec_unbound_parameter_launches_nothing);
    }
    std::printf("OK: %d failed\n", g_failed);
    return g_failed ? 1 : 0;
}
