// rhizome_delta.cpp -- crates/ops/src/delta.rs's API over librhizome_gdr.so.
//
// Every call: check lengths as the reference's slicing would (throwing where
// it would panic), convert to fp32, copy to device memory, launch through the
// C ABI on the default stream, copy back, widen to f64.

#include "rhizome_delta.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "rhizome_gdr.h"

namespace rhizome {
namespace ops {
namespace {

[[noreturn]] void fail(int32_t status, const std::string& what) { throw Error(status, what); }

void check(int32_t status, const char* call) {
    if (status != RHZ_OK)
        fail(status, std::string(call) + ": " + rhz_status_string(status) + ": " + rhz_last_error());
}

void hip_check(hipError_t e, const char* call) {
    if (e != hipSuccess) fail(RHZ_ERR_HIP, std::string(call) + ": " + hipGetErrorString(e));
}

void require(bool ok, const std::string& what) {
    if (!ok) fail(RHZ_ERR_INVALID_ARG, what);
}

// Device allocation owned for the duration of one call.
class DevBuf {
public:
    explicit DevBuf(std::size_t bytes) {
        if (bytes) hip_check(hipMalloc(&p_, bytes), "hipMalloc");
    }
    ~DevBuf() {
        if (p_) (void)hipFree(p_);
    }
    DevBuf(DevBuf&& o) noexcept : p_(o.p_) { o.p_ = nullptr; }
    DevBuf(const DevBuf&) = delete;
    DevBuf& operator=(const DevBuf&) = delete;
    template <typename T>
    T* as() const {
        return static_cast<T*>(p_);
    }

private:
    void* p_ = nullptr;
};

DevBuf upload_f32(const double* x, std::size_t n) {
    std::vector<float> h(x, x + n);
    DevBuf b(n * sizeof(float));
    if (n) hip_check(hipMemcpy(b.as<void>(), h.data(), n * sizeof(float), hipMemcpyHostToDevice), "hipMemcpy");
    return b;
}

std::vector<double> download_f64(const float* dev, std::size_t n) {
    std::vector<float> h(n);
    if (n) hip_check(hipMemcpy(h.data(), dev, n * sizeof(float), hipMemcpyDeviceToHost), "hipMemcpy");
    return std::vector<double>(h.begin(), h.end());
}

// The lengths delta.rs's loops index, for T positions of width d.
void require_inputs(const DeltaInputs& inp, std::size_t t, std::size_t d, const char* fn) {
    const std::string f(fn);
    require(inp.q.size() >= t * d, f + ": q holds fewer than T x head_dim values");
    require(inp.k.size() >= t * d, f + ": k holds fewer than T x head_dim values");
    require(inp.v.size() >= t * d, f + ": v holds fewer than T x head_dim values");
    require(inp.beta.size() >= t, f + ": beta is shorter than alpha");
    require(inp.segment.size() >= t, f + ": segment is shorter than alpha");
}

// Packed-sequence offsets: a new sequence wherever the segment id changes.
std::vector<int32_t> segment_offsets(const std::vector<std::size_t>& segment, std::size_t t) {
    std::vector<int32_t> cu{0};
    for (std::size_t i = 1; i < t; ++i)
        if (segment[i] != segment[i - 1]) cu.push_back(static_cast<int32_t>(i));
    cu.push_back(static_cast<int32_t>(t));
    return cu;
}

std::pair<std::vector<double>, DeltaState> run_sequence(const DeltaInputs& inp, const DeltaState& init,
                                                        std::size_t chunk, const char* fn) {
    const std::size_t t = inp.len(), d = inp.head_dim;
    if (t == 0) return {std::vector<double>{}, init};  // no position, no reset
    require(init.head_dim == d, std::string(fn) + ": init.head_dim differs from inputs.head_dim");
    require_inputs(inp, t, d, fn);
    if (d == 0) return {std::vector<double>{}, DeltaState::zeros(0)};
    require(t <= static_cast<std::size_t>(INT32_MAX), std::string(fn) + ": too many positions");

    const std::vector<int32_t> cu = segment_offsets(inp.segment, t);
    const std::size_t n_seq = cu.size() - 1;
    DevBuf q = upload_f32(inp.q.data(), t * d), k = upload_f32(inp.k.data(), t * d),
           v = upload_f32(inp.v.data(), t * d);
    DevBuf a = upload_f32(inp.alpha.data(), t), b = upload_f32(inp.beta.data(), t);
    DevBuf cu_dev(cu.size() * sizeof(int32_t));
    hip_check(hipMemcpy(cu_dev.as<void>(), cu.data(), cu.size() * sizeof(int32_t), hipMemcpyHostToDevice),
              "hipMemcpy");
    DevBuf o(t * d * sizeof(float)), fin(n_seq * d * d * sizeof(float));

    rhz_gdr_prefill_args args{};
    args.batch = static_cast<int32_t>(n_seq);
    args.seq_len = static_cast<int32_t>(t);
    args.heads = 1;
    args.d_k = args.d_v = static_cast<int32_t>(d);
    args.chunk = static_cast<int32_t>(std::min<std::size_t>(std::max<std::size_t>(chunk, 1), INT32_MAX));
    args.dtype = RHZ_F32;
    args.gate_kind = RHZ_GATE_ALPHA;
    args.algo = RHZ_ALGO_AUTO;
    args.q = q.as<void>();
    args.k = k.as<void>();
    args.v = v.as<void>();
    args.gate = a.as<float>();
    args.beta = b.as<float>();
    args.cu_seqlens = cu_dev.as<int32_t>();
    args.initial_state = nullptr;  // the reference resets at t = 0
    args.final_state = fin.as<float>();
    args.o = o.as<void>();
    std::size_t ws_bytes = 0;
    check(rhz_gdr_prefill_workspace_size(&args, &ws_bytes), "rhz_gdr_prefill_workspace_size");
    DevBuf ws(ws_bytes);
    args.workspace = ws.as<void>();
    args.workspace_bytes = ws_bytes;
    check(rhz_gdr_prefill(&args, nullptr), "rhz_gdr_prefill");

    std::vector<double> out = download_f64(o.as<float>(), t * d);
    DeltaState last{d, download_f64(fin.as<float>() + (n_seq - 1) * d * d, d * d)};
    return {std::move(out), std::move(last)};
}

}  // namespace

bool DeltaInputs::is_consistent() const {
    const std::size_t t = len(), d = head_dim;
    return d > 0 && q.size() == t * d && k.size() == t * d && v.size() == t * d && beta.size() == t &&
           segment.size() == t;
}

DeltaState DeltaState::zeros(std::size_t head_dim) { return DeltaState{head_dim, std::vector<double>(head_dim * head_dim, 0.0)}; }

void DeltaState::reset() { std::fill(s.begin(), s.end(), 0.0); }

double DeltaState::max_abs_diff(const DeltaState& other) const {
    double m = 0.0;
    const std::size_t n = std::min(s.size(), other.s.size());
    for (std::size_t i = 0; i < n; ++i) m = std::max(m, std::fabs(s[i] - other.s[i]));
    return m;
}

std::vector<double> gated_delta_step(DeltaState& state, const std::vector<double>& q,
                                     const std::vector<double>& k, const std::vector<double>& v,
                                     double alpha, double beta) {
    const std::size_t d = state.head_dim;
    require(state.s.size() >= d * d, "gated_delta_step: state.s holds fewer than head_dim^2 values");
    require(q.size() >= d && k.size() >= d && v.size() >= d,
            "gated_delta_step: q, k and v need head_dim values each");
    if (d == 0) return {};
    DevBuf qd = upload_f32(q.data(), d), kd = upload_f32(k.data(), d), vd = upload_f32(v.data(), d);
    DevBuf ad = upload_f32(&alpha, 1), bd = upload_f32(&beta, 1);
    DevBuf sd = upload_f32(state.s.data(), d * d);
    DevBuf od(d * sizeof(float));
    rhz_gdr_decode_args args{};
    args.batch = args.heads = 1;
    args.d_k = args.d_v = static_cast<int32_t>(d);
    args.dtype = RHZ_F32;
    args.gate_kind = RHZ_GATE_ALPHA;
    args.q = qd.as<void>();
    args.k = kd.as<void>();
    args.v = vd.as<void>();
    args.gate = ad.as<float>();
    args.beta = bd.as<float>();
    args.state = sd.as<float>();
    args.o = od.as<void>();
    check(rhz_gdr_decode_step(&args, nullptr), "rhz_gdr_decode_step");
    const std::vector<double> s = download_f64(sd.as<float>(), d * d);
    std::copy(s.begin(), s.end(), state.s.begin());
    return download_f64(od.as<float>(), d);
}

std::pair<std::vector<double>, DeltaState> gated_delta_sequential(const DeltaInputs& inp, const DeltaState& init) {
    return run_sequence(inp, init, 64, "gated_delta_sequential");
}

std::pair<std::vector<double>, DeltaState> gated_delta_scan_chunked(const DeltaInputs& inp, const DeltaState& init,
                                                                    std::size_t chunk) {
    return run_sequence(inp, init, chunk, "gated_delta_scan_chunked");
}

std::pair<std::vector<double>, std::vector<DeltaState>> gated_delta_multistep(const DeltaInputs& inp,
                                                                             const DeltaState& init,
                                                                             std::size_t max_positions) {
    const std::size_t d = inp.head_dim, n = std::min(inp.len(), max_positions);
    if (n == 0) return {};
    require(init.head_dim == d, "gated_delta_multistep: init.head_dim differs from inputs.head_dim");
    require_inputs(inp, n, d, "gated_delta_multistep");
    if (d == 0) return {std::vector<double>{}, std::vector<DeltaState>(n, DeltaState::zeros(0))};

    // reset at t = 0 (a zero state) and alpha = 0 wherever the segment changes
    std::vector<double> alpha(inp.alpha.begin(), inp.alpha.begin() + n);
    for (std::size_t t = 1; t < n; ++t)
        if (inp.segment[t] != inp.segment[t - 1]) alpha[t] = 0.0;
    DevBuf q = upload_f32(inp.q.data(), n * d), k = upload_f32(inp.k.data(), n * d),
           v = upload_f32(inp.v.data(), n * d);
    DevBuf a = upload_f32(alpha.data(), n), b = upload_f32(inp.beta.data(), n);
    const std::vector<double> zero(d * d, 0.0);
    DevBuf s0 = upload_f32(zero.data(), d * d);
    DevBuf snaps(n * d * d * sizeof(float)), o(n * d * sizeof(float));
    // windows of at most RHZ_MULTISTEP_MAX positions, each starting from the
    // previous window's last snapshot
    for (std::size_t t0 = 0; t0 < n; t0 += RHZ_MULTISTEP_MAX) {
        const std::size_t m = std::min<std::size_t>(RHZ_MULTISTEP_MAX, n - t0);
        rhz_gdr_multistep_args args{};
        args.batch = args.heads = 1;
        args.steps = static_cast<int32_t>(m);
        args.d_k = args.d_v = static_cast<int32_t>(d);
        args.dtype = RHZ_F32;
        args.gate_kind = RHZ_GATE_ALPHA;
        args.q = q.as<float>() + t0 * d;
        args.k = k.as<float>() + t0 * d;
        args.v = v.as<float>() + t0 * d;
        args.gate = a.as<float>() + t0;
        args.beta = b.as<float>() + t0;
        args.state = t0 == 0 ? s0.as<float>() : snaps.as<float>() + (t0 - 1) * d * d;
        args.states = snaps.as<float>() + t0 * d * d;
        args.o = o.as<float>() + t0 * d;
        check(rhz_gdr_multistep(&args, nullptr), "rhz_gdr_multistep");
    }
    const std::vector<double> all = download_f64(snaps.as<float>(), n * d * d);
    std::vector<DeltaState> states;
    states.reserve(n);
    for (std::size_t t = 0; t < n; ++t)
        states.push_back(DeltaState{d, std::vector<double>(all.begin() + t * d * d, all.begin() + (t + 1) * d * d)});
    return {download_f64(o.as<float>(), n * d), std::move(states)};
}

}  // namespace ops
}  // namespace rhizome
