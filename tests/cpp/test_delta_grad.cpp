// Tests of the f64 adjoint of the gated delta rule
// (rhizome_amd/host/rhizome_delta_grad.hpp).  CPU only: the backward has no
// GPU path.
//
// The adjoint is held to central differences of the f64 oracle's forward
// (oracle/gdr_oracle.c, the restatement of delta.rs:94-154) under the
// reference's gradient-check rule (gradcheck.rs:33-53: h = 1e-5, relative
// error <= 1e-6, docs/kernels.md:28-30), with the loss
// L = <W_o, o> + <W_S, final state> for fixed random weights.  Exact
// identities pin what differences cannot: o is linear in v (zero initial
// state) and in q, so <W_o, o> equals <dv, v> and <dq, q>; a reset cuts every
// gradient before it to exactly zero.
//
// Exit status 0 when every test passes.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

#include "rhizome_delta_grad.hpp"
#include "rhizome_gdr.h"

using namespace rhizome::ops;

// The f64 oracle (oracle/gdr_oracle.c), test infrastructure only.
extern "C" {
void orc_make_inputs(int64_t t_len, int64_t d, uint64_t seed, double* q, double* k, double* v, double* alpha,
                     double* beta);
void orc_gated_delta_sequential(int64_t t_len, int64_t d, const double* q, const double* k, const double* v,
                                const double* alpha, const double* beta, const uint64_t* segment,
                                const double* init, double* out, double* final_state);
void orc_gdr_prefill_batched(int64_t n_seqs, const int64_t* cu_seqlens, int64_t heads, int64_t dk, int64_t dv,
                             const double* q, const double* k, const double* v, const double* alpha,
                             const double* beta, const double* init, double* o, double* final_state,
                             int nthreads);
void orc_philox_normal(uint64_t seed, uint64_t stream, int64_t n, double mean, double std_, double* out,
                       int nthreads);
void orc_l2norm_rows(double* x, int64_t rows, int64_t d, double scale, int nthreads);
void orc_sigmoid_vec(const double* z, int64_t n, double* out);
void orc_neg_softplus_vec(const double* z, int64_t n, double* out);
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

constexpr double kRtol = 1e-6;  // docs/kernels.md:30

std::vector<double> normal(uint64_t seed, uint64_t stream, std::size_t n, double mean = 0.0, double sd = 1.0) {
    std::vector<double> x(n);
    orc_philox_normal(seed, stream, int64_t(n), mean, sd, x.data(), 1);
    return x;
}

double dot(const std::vector<double>& a, const std::vector<double>& b) {
    double s = 0.0;
    for (std::size_t i = 0; i < a.size(); ++i) s += a[i] * b[i];
    return s;
}

void expect_check(const char* what, const std::function<double(const std::vector<double>&)>& f,
                  const std::vector<double>& x, const std::vector<double>& analytic) {
    EXPECT(x.size() == analytic.size());
    const gradcheck::GradCheckReport r = gradcheck::check(f, x, analytic);
    std::printf("  %-8s n=%-4zu max rel err %.2e at %zu (analytic %.3e)\n", what, x.size(), r.max_rel_err,
                r.worst_index, analytic[r.worst_index]);
    if (!r.passes(kRtol))
        throw std::runtime_error(std::string(what) + ": max relative error " + std::to_string(r.max_rel_err) +
                                 " at index " + std::to_string(r.worst_index));
}

// ------------------------------------------------------------ gradcheck.rs tests
void gradcheck_detects_a_correct_gradient() {  // gradcheck.rs:59-64
    const std::vector<double> x{0.3, -1.7, 2.2};
    std::vector<double> an;
    for (double v : x) an.push_back(2.0 * v);
    auto f = [](const std::vector<double>& v) { return dot(v, v); };
    EXPECT(gradcheck::check(f, x, an).passes(1e-6));
}

void gradcheck_detects_an_incorrect_gradient() {  // gradcheck.rs:66-73
    const std::vector<double> x{0.3, -1.7};
    auto f = [](const std::vector<double>& v) { return dot(v, v); };
    const auto r = gradcheck::check(f, x, {0.0, 0.0});
    EXPECT(!r.passes(1e-6) && r.max_rel_err > 0.5);
}

// ------------------------------------------------------------ one head (delta.rs signature)
struct Seq {
    DeltaInputs inp;
    std::vector<double> wo, wf;  // loss weights
};

Seq make_seq(std::size_t t, std::size_t d, const std::vector<std::size_t>& segs, uint64_t seed) {
    Seq s;
    s.inp.head_dim = d;
    s.inp.q.resize(t * d);
    s.inp.k.resize(t * d);
    s.inp.v.resize(t * d);
    s.inp.alpha.resize(t);
    s.inp.beta.resize(t);
    orc_make_inputs(t, d, seed, s.inp.q.data(), s.inp.k.data(), s.inp.v.data(), s.inp.alpha.data(), s.inp.beta.data());
    s.inp.segment = segs;
    s.wo = normal(seed, 40, t * d);
    s.wf = normal(seed, 41, d * d);
    return s;
}

// L = <W_o, o> + <W_S, final> through the oracle's forward.
double seq_loss(const DeltaInputs& in, const std::vector<double>& wo, const std::vector<double>& wf) {
    const std::size_t t = in.len(), d = in.head_dim;
    std::vector<double> o(t * d), fin(d * d), init(d * d, 0.0);
    std::vector<uint64_t> seg(in.segment.begin(), in.segment.end());
    orc_gated_delta_sequential(t, d, in.q.data(), in.k.data(), in.v.data(), in.alpha.data(), in.beta.data(), seg.data(),
                               init.data(), o.data(), fin.data());
    return dot(wo, o) + dot(wf, fin);
}

void check_sequence(const Seq& s) {
    DeltaState dfin;
    dfin.head_dim = s.inp.head_dim;
    dfin.s = s.wf;
    const DeltaGrads g = gated_delta_sequential_backward(s.inp, DeltaState::zeros(s.inp.head_dim), s.wo, &dfin);
    auto field = [&](std::vector<double> DeltaInputs::*m, const std::vector<double>& an, const char* what) {
        expect_check(what,
                     [&](const std::vector<double>& x) {
                         DeltaInputs in = s.inp;
                         in.*m = x;
                         return seq_loss(in, s.wo, s.wf);
                     },
                     s.inp.*m, an);
    };
    field(&DeltaInputs::q, g.q, "dq");
    field(&DeltaInputs::k, g.k, "dk");
    field(&DeltaInputs::v, g.v, "dv");
    field(&DeltaInputs::alpha, g.alpha, "dalpha");
    field(&DeltaInputs::beta, g.beta, "dbeta");
    for (double x : g.init.s) EXPECT(x == 0.0);  // t = 0 resets: init never reaches the loss
}

void sequential_single_segment() { check_sequence(make_seq(12, 4, std::vector<std::size_t>(12, 0), 2)); }

void sequential_with_segments() {  // the segment layout of delta.rs:305-317
    check_sequence(make_seq(10, 4, {0, 0, 0, 1, 1, 2, 2, 2, 2, 3}, 3));
}

void sequential_across_windows() {  // 150 positions: three windows of the reverse scan
    std::vector<std::size_t> segs(150, 0);
    for (std::size_t t = 100; t < 150; ++t) segs[t] = 1;
    check_sequence(make_seq(150, 3, segs, 4));
}

void empty_sequence_passes_d_final_to_init() {
    Seq s = make_seq(0, 3, {}, 5);
    DeltaState dfin;
    dfin.head_dim = 3;
    dfin.s = normal(5, 41, 9);
    const DeltaGrads g = gated_delta_sequential_backward(s.inp, DeltaState::zeros(3), {}, &dfin);
    EXPECT(g.q.empty() && g.alpha.empty() && g.init.s == dfin.s);
}

void linear_in_v_and_q() {
    const Seq s = make_seq(40, 5, std::vector<std::size_t>(40, 0), 6);
    const DeltaGrads g = gated_delta_sequential_backward(s.inp, DeltaState::zeros(5), s.wo, nullptr);
    std::vector<double> o(40 * 5), fin(25), init(25, 0.0);
    std::vector<uint64_t> seg(40, 0);
    orc_gated_delta_sequential(40, 5, s.inp.q.data(), s.inp.k.data(), s.inp.v.data(), s.inp.alpha.data(),
                               s.inp.beta.data(), seg.data(), init.data(), o.data(), fin.data());
    const double l = dot(s.wo, o), lv = dot(g.v, s.inp.v), lq = dot(g.q, s.inp.q);
    std::printf("  <W,o> %.15g  <dv,v> %.15g  <dq,q> %.15g\n", l, lv, lq);
    EXPECT(std::fabs(l - lv) <= 1e-12 * std::fabs(l) + 1e-12);
    EXPECT(std::fabs(l - lq) <= 1e-12 * std::fabs(l) + 1e-12);
}

void reset_cuts_gradients() {
    Seq s = make_seq(9, 4, {0, 0, 0, 0, 1, 1, 1, 1, 1}, 7);
    for (std::size_t i = 0; i < 4 * 4; ++i) s.wo[i] = 0.0;  // no loss on the first segment's outputs
    DeltaState dfin;
    dfin.head_dim = 4;
    dfin.s = s.wf;
    const DeltaGrads g = gated_delta_sequential_backward(s.inp, DeltaState::zeros(4), s.wo, &dfin);
    for (std::size_t t = 0; t < 4; ++t) {
        EXPECT(g.alpha[t] == 0.0 && g.beta[t] == 0.0);
        for (std::size_t j = 0; j < 4; ++j) EXPECT(g.q[t * 4 + j] == 0.0 && g.k[t * 4 + j] == 0.0 && g.v[t * 4 + j] == 0.0);
    }
    bool any = false;
    for (std::size_t t = 4; t < 9; ++t) any |= g.beta[t] != 0.0;
    EXPECT(any);
}

void inconsistent_lengths_throw() {
    Seq s = make_seq(6, 3, std::vector<std::size_t>(6, 0), 8);
    s.inp.beta.pop_back();
    bool thrown = false;
    try {
        gated_delta_sequential_backward(s.inp, DeltaState::zeros(3), s.wo, nullptr);
    } catch (const Error& e) {
        thrown = e.status() == RHZ_ERR_INVALID_ARG;
    }
    EXPECT(thrown);
}

// ------------------------------------------------------------ batched prefill
// Packed sequences of lengths 5, 0 and 70 (past one window), H = 2,
// d_k = 3, d_v = 5, honoured initial states; with log-decay and alpha gates.
// Returns the gate gradient.  With log-decay gates, d g = d alpha * alpha is
// smaller than the finite-difference noise of this loss at some positions
// (|d g| ~ 1e-4 against ~5e-10), so it is pinned by that identity against
// the checked alpha-gate gradient instead (batched_log_gate_is_chain_rule).
std::vector<double> batched_packed(int gate_kind) {
    const std::vector<int64_t> cu{0, 5, 5, 75};
    const std::size_t N = 3, H = 2, dk = 3, dv = 5, tok = 75, seed = 9;
    std::vector<double> q = normal(seed, 1, tok * H * dk), k = normal(seed, 2, tok * H * dk);
    orc_l2norm_rows(q.data(), tok * H, dk, 1.0, 1);
    orc_l2norm_rows(k.data(), tok * H, dk, 1.0, 1);
    std::vector<double> v = normal(seed, 3, tok * H * dv), beta(tok * H), gate(tok * H);
    const std::vector<double> zb = normal(seed, 4, tok * H), zg = normal(seed, 5, tok * H);
    orc_sigmoid_vec(zb.data(), tok * H, beta.data());
    orc_neg_softplus_vec(zg.data(), tok * H, gate.data());  // log-decay g
    if (gate_kind == RHZ_GATE_ALPHA)
        for (double& x : gate) x = std::exp(x);
    const std::vector<double> init = normal(seed, 6, N * H * dv * dk, 0.0, 0.5);
    const std::vector<double> wo = normal(seed, 40, tok * H * dv), wf = normal(seed, 41, N * H * dv * dk);

    auto loss = [&](const std::vector<double>& q_, const std::vector<double>& k_, const std::vector<double>& v_,
                    const std::vector<double>& g_, const std::vector<double>& b_, const std::vector<double>& s_) {
        std::vector<double> alpha(g_);
        if (gate_kind == RHZ_GATE_LOG_ALPHA)
            for (double& x : alpha) x = std::exp(x);
        std::vector<double> o(tok * H * dv), fin(N * H * dv * dk);
        orc_gdr_prefill_batched(N, cu.data(), H, dk, dv, q_.data(), k_.data(), v_.data(), alpha.data(), b_.data(),
                                s_.data(), o.data(), fin.data(), 1);
        return dot(wo, o) + dot(wf, fin);
    };
    std::vector<double> dq(q.size()), dk_(k.size()), dv_(v.size()), dg(gate.size()), db(beta.size()), ds(init.size());
    PrefillBackwardArgs a;
    a.batch = N;
    a.seq_len = tok;
    a.heads = H;
    a.d_k = dk;
    a.d_v = dv;
    a.gate_kind = gate_kind;
    a.q = q.data();
    a.k = k.data();
    a.v = v.data();
    a.gate = gate.data();
    a.beta = beta.data();
    a.cu_seqlens = cu.data();
    a.initial_state = init.data();
    a.d_o = wo.data();
    a.d_final_state = wf.data();
    a.dq = dq.data();
    a.dk = dk_.data();
    a.dv = dv_.data();
    a.dgate = dg.data();
    a.dbeta = db.data();
    a.d_initial_state = ds.data();
    a.threads = 3;
    gated_delta_prefill_backward(a);
    expect_check("dq", [&](const std::vector<double>& x) { return loss(x, k, v, gate, beta, init); }, q, dq);
    expect_check("dk", [&](const std::vector<double>& x) { return loss(q, x, v, gate, beta, init); }, k, dk_);
    expect_check("dv", [&](const std::vector<double>& x) { return loss(q, k, x, gate, beta, init); }, v, dv_);
    if (gate_kind == RHZ_GATE_ALPHA)
        expect_check("dgate", [&](const std::vector<double>& x) { return loss(q, k, v, x, beta, init); }, gate, dg);
    expect_check("dbeta", [&](const std::vector<double>& x) { return loss(q, k, v, gate, x, init); }, beta, db);
    expect_check("dinit", [&](const std::vector<double>& x) { return loss(q, k, v, gate, beta, x); }, init, ds);
    // The empty sequence's state passes through: d init = d final.
    for (std::size_t i = H * dv * dk; i < 2 * H * dv * dk; ++i) EXPECT(ds[i] == wf[i]);
    return dg;
}

void batched_log_gate_is_chain_rule() {
    const std::vector<double> dg_log = batched_packed(RHZ_GATE_LOG_ALPHA);
    const std::vector<double> dalpha = batched_packed(RHZ_GATE_ALPHA);
    // The same gates: alpha = exp(g) with g from the same stream.
    std::vector<double> g(dg_log.size());
    const std::vector<double> zg = normal(9, 5, g.size());
    orc_neg_softplus_vec(zg.data(), int64_t(g.size()), g.data());
    for (std::size_t i = 0; i < g.size(); ++i) EXPECT(dg_log[i] == dalpha[i] * std::exp(g[i]));
}

void batched_threads_agree() {  // the thread count does not change a bit
    const std::size_t B = 3, T = 20, H = 4, d = 4;
    std::vector<double> q = normal(1, 1, B * T * H * d), k = normal(1, 2, B * T * H * d);
    orc_l2norm_rows(k.data(), B * T * H, d, 1.0, 1);
    const std::vector<double> v = normal(1, 3, B * T * H * d), g = normal(1, 5, B * T * H, -1.0, 0.1);
    const std::vector<double> b(B * T * H, 0.5), wo = normal(1, 40, B * T * H * d);
    std::vector<double> out[2][5];
    for (int r = 0; r < 2; ++r) {
        for (auto& x : out[r]) x.assign(B * T * H * d, 0.0);
        PrefillBackwardArgs a;
        a.batch = B;
        a.seq_len = T;
        a.heads = H;
        a.d_k = a.d_v = d;
        a.q = q.data();
        a.k = k.data();
        a.v = v.data();
        a.gate = g.data();
        a.beta = b.data();
        a.d_o = wo.data();
        a.dq = out[r][0].data();
        a.dk = out[r][1].data();
        a.dv = out[r][2].data();
        a.dgate = out[r][3].data();
        a.dbeta = out[r][4].data();
        a.threads = r == 0 ? 1 : 8;
        gated_delta_prefill_backward(a);
    }
    for (int i = 0; i < 5; ++i) EXPECT(out[0][i] == out[1][i]);
}

// The batched form on a dense batch with zero initial states, head by head,
// equals the one-head form (which resets at t = 0), bit for bit: the same
// reverse scan over strided rows.
void batched_equals_one_head() {
    const std::size_t B = 2, T = 130, H = 3, d = 8, rows = B * T * H;
    std::vector<double> q = normal(3, 1, rows * d), k = normal(3, 2, rows * d);
    orc_l2norm_rows(q.data(), rows, d, 1.0, 1);
    orc_l2norm_rows(k.data(), rows, d, 1.0, 1);
    const std::vector<double> v = normal(3, 3, rows * d), wo = normal(3, 40, rows * d), wf = normal(3, 41, B * H * d * d);
    std::vector<double> alpha(rows), beta(rows);
    const std::vector<double> za = normal(3, 5, rows), zb = normal(3, 4, rows);
    orc_sigmoid_vec(zb.data(), rows, beta.data());
    orc_sigmoid_vec(za.data(), rows, alpha.data());
    std::vector<double> dq(rows * d), dk(rows * d), dv(rows * d), da(rows), db(rows);
    PrefillBackwardArgs a;
    a.batch = B;
    a.seq_len = T;
    a.heads = H;
    a.d_k = a.d_v = d;
    a.gate_kind = RHZ_GATE_ALPHA;
    a.q = q.data();
    a.k = k.data();
    a.v = v.data();
    a.gate = alpha.data();
    a.beta = beta.data();
    a.d_o = wo.data();
    a.d_final_state = wf.data();
    a.dq = dq.data();
    a.dk = dk.data();
    a.dv = dv.data();
    a.dgate = da.data();
    a.dbeta = db.data();
    a.threads = 4;
    gated_delta_prefill_backward(a);
    for (std::size_t b = 0; b < B; ++b)
        for (std::size_t h = 0; h < H; ++h) {
            DeltaInputs in;
            in.head_dim = d;
            std::vector<double> w_o(T * d);
            for (std::size_t t = 0; t < T; ++t) {
                const std::size_t r = (b * T + t) * H + h;
                in.q.insert(in.q.end(), q.begin() + r * d, q.begin() + (r + 1) * d);
                in.k.insert(in.k.end(), k.begin() + r * d, k.begin() + (r + 1) * d);
                in.v.insert(in.v.end(), v.begin() + r * d, v.begin() + (r + 1) * d);
                in.alpha.push_back(alpha[r]);
                in.beta.push_back(beta[r]);
                in.segment.push_back(0);
                std::copy(wo.begin() + r * d, wo.begin() + (r + 1) * d, w_o.begin() + t * d);
            }
            DeltaState dfin;
            dfin.head_dim = d;
            dfin.s.assign(wf.begin() + (b * H + h) * d * d, wf.begin() + (b * H + h + 1) * d * d);
            const DeltaGrads g = gated_delta_sequential_backward(in, DeltaState::zeros(d), w_o, &dfin);
            for (std::size_t t = 0; t < T; ++t) {
                const std::size_t r = (b * T + t) * H + h;
                EXPECT(g.alpha[t] == da[r] && g.beta[t] == db[r]);
                for (std::size_t j = 0; j < d; ++j)
                    EXPECT(g.q[t * d + j] == dq[r * d + j] && g.k[t * d + j] == dk[r * d + j] && g.v[t * d + j] == dv[r * d + j]);
            }
        }
}

}  // namespace

int main() {
    run("gradcheck_detects_a_correct_gradient", gradcheck_detects_a_correct_gradient);
    run("gradcheck_detects_an_incorrect_gradient", gradcheck_detects_an_incorrect_gradient);
    run("sequential_single_segment", sequential_single_segment);
    run("sequential_with_segments", sequential_with_segments);
    run("sequential_across_windows", sequential_across_windows);
    run("empty_sequence_passes_d_final_to_init", empty_sequence_passes_d_final_to_init);
    run("linear_in_v_and_q", linear_in_v_and_q);
    run("reset_cuts_gradients", reset_cuts_gradients);
    run("inconsistent_lengths_throw", inconsistent_lengths_throw);
    run("batched_packed_alpha_gate", [] { batched_packed(RHZ_GATE_ALPHA); });
    run("batched_log_gate_is_chain_rule", batched_log_gate_is_chain_rule);
    run("batched_threads_agree", batched_threads_agree);
    run("batched_equals_one_head", batched_equals_one_head);
    std::printf("OK: %d failed\n", g_failed);
    return g_failed ? 1 : 0;
}
