// Tests of the C++ restatement of crates/ops/src/delta.rs (rhizome_amd/host),
// which runs on the GPU through librhizome_gdr.so.  The first group follows
// the reference's own unit tests (delta.rs:282-358, same inputs from the
// reference's fixture builder, delta.rs:254-280, via the f64 oracle), with
// tolerances widened from the reference's f64 1e-10 / 1e-12 to what fp32
// on the device gives; the second compares each function with the f64 oracle
// (the CPU restatement of delta.rs) on the same inputs; the third checks the
// error behaviour, which needs no GPU.
//
//   test_delta_host            every test (needs a GPU)
//   test_delta_host --cpu      the tests that make no GPU call
//
// Exit status 0 when every test passes.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

#include "rhizome_delta.hpp"
#include "rhizome_gdr.h"

using namespace rhizome::ops;

// The f64 oracle (oracle/gdr_oracle.c), test infrastructure only.
extern "C" {
void orc_make_inputs(int64_t t_len, int64_t d, uint64_t seed, double* q, double* k, double* v, double* alpha,
                     double* beta);
void orc_gated_delta_sequential(int64_t t_len, int64_t d, const double* q, const double* k, const double* v,
                                const double* alpha, const double* beta, const uint64_t* segment,
                                const double* init, double* out, double* final_state);
int64_t orc_gated_delta_multistep(int64_t t_len, int64_t d, const double* q, const double* k, const double* v,
                                  const double* alpha, const double* beta, const uint64_t* segment,
                                  const double* init, int64_t max_positions, double* outs, double* states);
double* orc_gated_delta_step(double* s, int64_t d, const double* q, const double* k, const double* v,
                             double alpha, double beta);
void orc_free(void* p);
}

namespace {

int g_failed = 0;

#define EXPECT(cond)                                                                 \
    do {                                                                             \
        if (!(cond)) throw std::runtime_error(std::string("expected: ") + #cond);    \
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

// delta.rs:254-280's fixture, built by the oracle's restatement of it.
DeltaInputs make_inputs(std::size_t t, std::size_t d, const std::vector<std::size_t>& segments, uint64_t seed) {
    DeltaInputs in;
    in.head_dim = d;
    in.q.resize(t * d);
    in.k.resize(t * d);
    in.v.resize(t * d);
    in.alpha.resize(t);
    in.beta.resize(t);
    orc_make_inputs(t, d, seed, in.q.data(), in.k.data(), in.v.data(), in.alpha.data(), in.beta.data());
    in.segment = segments;
    return in;
}

std::vector<std::size_t> segs_zero(std::size_t t) { return std::vector<std::size_t>(t, 0); }

// fp32 device results against f64: |x - y| <= 1e-4 (RMS(y) + |y|).
void expect_close(const std::vector<double>& x, const std::vector<double>& y, const char* what) {
    EXPECT(x.size() == y.size());
    double ss = 0.0;
    for (double v : y) ss += v * v;
    const double rms = y.empty() ? 0.0 : std::sqrt(ss / y.size());
    for (std::size_t i = 0; i < x.size(); ++i)
        if (!(std::fabs(x[i] - y[i]) <= 1e-4 * (rms + std::fabs(y[i]))))
            throw std::runtime_error(std::string(what) + ": element " + std::to_string(i) + " " +
                                     std::to_string(x[i]) + " vs " + std::to_string(y[i]));
}

std::vector<uint64_t> u64(const std::vector<std::size_t>& s) { return std::vector<uint64_t>(s.begin(), s.end()); }

// ---------------------------------------------------------------- reference tests
void inputs_validate_shapes() {  // delta.rs:282-287
    DeltaInputs inp = make_inputs(4, 3, {0, 0, 0, 0}, 1);
    EXPECT(inp.is_consistent());
    EXPECT(!inp.is_empty());
    inp.beta.pop_back();
    EXPECT(!inp.is_consistent());
    DeltaInputs none;
    EXPECT(!none.is_consistent());  // head_dim 0
    EXPECT(none.is_empty());
}

void chunked_matches_sequential_single_segment() {  // delta.rs:289-303
    const std::size_t t = 40, d = 6;
    const DeltaInputs inp = make_inputs(t, d, segs_zero(t), 2);
    const DeltaState init = DeltaState::zeros(d);
    const auto [a, sa] = gated_delta_sequential(inp, init);
    for (std::size_t chunk : {1, 3, 8, 64}) {
        const auto [b, sb] = gated_delta_scan_chunked(inp, init, chunk);
        for (std::size_t i = 0; i < a.size(); ++i) EXPECT(std::fabs(a[i] - b[i]) < 1e-10);
        EXPECT(sa.max_abs_diff(sb) < 1e-10);
    }
}

void chunked_matches_sequential_with_segments() {  // delta.rs:305-317
    const std::size_t d = 4;
    const std::vector<std::size_t> segs{0, 0, 0, 1, 1, 2, 2, 2, 2, 3};
    const DeltaInputs inp = make_inputs(segs.size(), d, segs, 3);
    const DeltaState init = DeltaState::zeros(d);
    const auto [a, sa] = gated_delta_sequential(inp, init);
    const auto [b, sb] = gated_delta_scan_chunked(inp, init, 4);
    for (std::size_t i = 0; i < a.size(); ++i) EXPECT(std::fabs(a[i] - b[i]) < 1e-10);
    EXPECT(sa.max_abs_diff(sb) < 1e-10);
}

void multistep_matches_repeated_step() {  // delta.rs:319-331 (multistep and sequence kernels: fp32)
    const std::size_t d = 5, t = 8;
    const DeltaInputs inp = make_inputs(t, d, segs_zero(t), 4);
    const DeltaState init = DeltaState::zeros(d);
    const auto [outs, states] = gated_delta_multistep(inp, init, 8);
    const auto [seq, final_state] = gated_delta_sequential(inp, init);
    EXPECT(states.size() == t);
    for (std::size_t i = 0; i < outs.size(); ++i) EXPECT(std::fabs(outs[i] - seq[i]) < 1e-5);
    EXPECT(states[t - 1].max_abs_diff(final_state) < 1e-5);
}

void segment_reset_makes_history_irrelevant() {  // delta.rs:333-346
    const std::size_t d = 3;
    const DeltaInputs inp = make_inputs(4, d, {0, 0, 1, 1}, 5);
    DeltaState dirty = DeltaState::zeros(d);
    for (double& v : dirty.s) v = 3.0;
    const auto [a, sa] = gated_delta_sequential(inp, DeltaState::zeros(d));
    const auto [b, sb] = gated_delta_sequential(inp, dirty);
    for (std::size_t i = 2 * d; i < 4 * d; ++i) EXPECT(std::fabs(a[i] - b[i]) < 1e-12);
}

void alpha_zero_forgets_the_past() {  // delta.rs:348-358
    const std::size_t d = 3;
    DeltaState s = DeltaState::zeros(d);
    for (double& v : s.s) v = 1.0;
    const std::vector<double> k{1.0, 0.0, 0.0}, v{0.0, 0.0, 0.0}, q{1.0, 1.0, 1.0};
    const std::vector<double> o = gated_delta_step(s, q, k, v, 0.0, 0.5);
    for (double x : o) EXPECT(std::fabs(x) < 1e-12);
}

// ---------------------------------------------------------------- against the oracle
void sequential_matches_oracle() {
    for (const auto& segs : std::vector<std::vector<std::size_t>>{
             segs_zero(200), {0, 0, 0, 1, 1, 2, 2, 2, 2, 3}, {7}, {1, 2, 1, 2, 1}}) {
        for (std::size_t d : {1, 6, 32, 128}) {
            const std::size_t t = segs.size();
            const DeltaInputs inp = make_inputs(t, d, segs, 11 + d);
            const DeltaState init = DeltaState::zeros(d);
            const auto [o, fin] = gated_delta_sequential(inp, init);
            std::vector<double> ro(t * d), rf(d * d);
            const std::vector<uint64_t> sg = u64(segs);
            orc_gated_delta_sequential(t, d, inp.q.data(), inp.k.data(), inp.v.data(), inp.alpha.data(),
                                       inp.beta.data(), sg.data(), init.s.data(), ro.data(), rf.data());
            expect_close(o, ro, "o");
            expect_close(fin.s, rf, "final state");
        }
    }
}

void multistep_matches_oracle() {
    // 150 positions: three device windows of at most 64
    const std::vector<std::size_t> segs = [] {
        std::vector<std::size_t> s(150, 0);
        for (std::size_t i = 70; i < 150; ++i) s[i] = 1;
        return s;
    }();
    const std::size_t d = 16;
    const DeltaInputs inp = make_inputs(segs.size(), d, segs, 21);
    const DeltaState init = DeltaState::zeros(d);
    for (std::size_t maxp : {std::size_t(1), std::size_t(8), std::size_t(150), std::size_t(1000)}) {
        const auto [o, states] = gated_delta_multistep(inp, init, maxp);
        const std::size_t n = std::min(maxp, segs.size());
        std::vector<double> ro(n * d), rs(n * d * d);
        const std::vector<uint64_t> sg = u64(segs);
        EXPECT(orc_gated_delta_multistep(segs.size(), d, inp.q.data(), inp.k.data(), inp.v.data(),
                                         inp.alpha.data(), inp.beta.data(), sg.data(), init.s.data(), maxp,
                                         ro.data(), rs.data()) == (int64_t)n);
        EXPECT(states.size() == n);
        expect_close(o, ro, "multistep o");
        for (std::size_t t = 0; t < n; ++t)
            expect_close(states[t].s, std::vector<double>(rs.begin() + t * d * d, rs.begin() + (t + 1) * d * d),
                         "multistep state");
    }
}

void step_matches_oracle() {
    const std::size_t d = 64;
    const DeltaInputs inp = make_inputs(5, d, segs_zero(5), 31);
    DeltaState s = DeltaState::zeros(d);
    std::vector<double> rs(d * d, 0.0);
    for (std::size_t t = 0; t < 5; ++t) {
        const std::vector<double> q(inp.q.begin() + t * d, inp.q.begin() + (t + 1) * d);
        const std::vector<double> k(inp.k.begin() + t * d, inp.k.begin() + (t + 1) * d);
        const std::vector<double> v(inp.v.begin() + t * d, inp.v.begin() + (t + 1) * d);
        const std::vector<double> o = gated_delta_step(s, q, k, v, inp.alpha[t], inp.beta[t]);
        double* ro = orc_gated_delta_step(rs.data(), d, q.data(), k.data(), v.data(), inp.alpha[t], inp.beta[t]);
        const std::vector<double> ref(ro, ro + d);
        orc_free(ro);
        expect_close(o, ref, "step o");
        expect_close(s.s, rs, "step state");
    }
}

void empty_inputs() {
    DeltaInputs inp;
    inp.head_dim = 4;
    DeltaState init = DeltaState::zeros(4);
    init.s[0] = 2.5;
    const auto [o, fin] = gated_delta_sequential(inp, init);  // no position: init comes back
    EXPECT(o.empty());
    EXPECT(fin.max_abs_diff(init) == 0.0 && fin.s.size() == 16);
    const auto [mo, ms] = gated_delta_multistep(inp, init, 8);
    EXPECT(mo.empty() && ms.empty());
}

// ---------------------------------------------------------------- errors (no GPU call)
void inconsistent_lengths_throw() {
    DeltaInputs inp = make_inputs(6, 4, segs_zero(6), 7);
    inp.v.resize(10);
    const DeltaState init = DeltaState::zeros(4);
    int thrown = 0;
    try {
        (void)gated_delta_sequential(inp, init);
    } catch (const Error& e) {
        thrown += e.status() == RHZ_ERR_INVALID_ARG && std::strstr(e.what(), "v holds") != nullptr;
    }
    try {
        (void)gated_delta_multistep(inp, DeltaState::zeros(3), 4);
    } catch (const Error& e) {
        thrown += e.status() == RHZ_ERR_INVALID_ARG && std::strstr(e.what(), "head_dim") != nullptr;
    }
    DeltaState s = DeltaState::zeros(4);
    try {
        (void)gated_delta_step(s, {1.0, 2.0}, inp.k, inp.v, 0.9, 0.5);
    } catch (const Error& e) {
        thrown += e.status() == RHZ_ERR_INVALID_ARG;
    }
    EXPECT(thrown == 3);
}

void state_helpers() {  // delta.rs:67-89
    DeltaState a = DeltaState::zeros(3), b = DeltaState::zeros(3);
    EXPECT(a.s.size() == 9 && a.max_abs_diff(b) == 0.0);
    b.s[4] = -2.0;
    b.s[7] = 0.5;
    EXPECT(a.max_abs_diff(b) == 2.0);
    b.reset();
    EXPECT(a.max_abs_diff(b) == 0.0);
}

}  // namespace

int main(int argc, char** argv) {
    const bool cpu_only = argc > 1 && std::strcmp(argv[1], "--cpu") == 0;
    run("inputs_validate_shapes", inputs_validate_shapes);
    run("state_helpers", state_helpers);
    run("inconsistent_lengths_throw", inconsistent_lengths_throw);
    run("empty_inputs", empty_inputs);
    if (!cpu_only) {
        run("chunked_matches_sequential_single_segment", chunked_matches_sequential_single_segment);
        run("chunked_matches_sequential_with_segments", chunked_matches_sequential_with_segments);
        run("multistep_matches_repeated_step", multistep_matches_repeated_step);
        run("segment_reset_makes_history_irrelevant", segment_reset_makes_history_irrelevant);
        run("alpha_zero_forgets_the_past", alpha_zero_forgets_the_past);
        run("sequential_matches_oracle", sequential_matches_oracle);
        run("multistep_matches_oracle", multistep_matches_oracle);
        run("step_matches_oracle", step_matches_oracle);
    }
    std::printf("%s: %d failed\n", g_failed ? "FAILED" : "OK", g_failed);
    return g_failed ? 1 : 0;
}
