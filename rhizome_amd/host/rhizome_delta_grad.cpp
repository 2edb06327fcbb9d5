// rhizome_delta_grad.cpp -- reverse scan of the gated delta rule (f64, CPU).

#include "rhizome_delta_grad.hpp"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <string>
#include <thread>

#include "rhizome_gdr.h"

namespace rhizome {
namespace ops {
namespace {

constexpr std::size_t kWindow = 64;  // positions between kept states

void require(bool ok, const std::string& what) {
    if (!ok) throw Error(RHZ_ERR_INVALID_ARG, what);
}

// One (sequence, head): position t reads q + t * qs, k + t * ks, v + t * vs,
// gate / beta + t * gs, d_o + t * os and writes the gradients at the same
// offsets.  reset[t] zeroes the state before position t.
struct Unit {
    std::size_t T = 0, dk = 0, dv = 0;
    const double *q, *k, *v, *gate, *beta, *d_o;
    std::size_t qs, ks, vs, gs, os;
    bool log_gate = false;
    const std::vector<char>* reset = nullptr;  // nullptr: no resets
    const double* init = nullptr;              // dv x dk, nullptr for zeros
    const double* d_final = nullptr;           // dv x dk, nullptr for zero
    double *dq, *dk_, *dv_, *dgate, *dbeta;
    double* dinit = nullptr;
};

// delta.rs:103-117 on a d_v x d_k state, in the reference's evaluation order.
void step(double* S, const double* k, const double* v, double a, double b, std::size_t dv, std::size_t dk,
          double* sk) {
    for (std::size_t i = 0; i < dv; ++i) {
        double acc = 0.0;
        for (std::size_t j = 0; j < dk; ++j) acc += S[i * dk + j] * k[j];
        sk[i] = acc;
    }
    for (std::size_t i = 0; i < dv; ++i)
        for (std::size_t j = 0; j < dk; ++j) {
            const double decayed = a * (S[i * dk + j] - b * sk[i] * k[j]);
            S[i * dk + j] = decayed + b * v[i] * k[j];
        }
}

void backward_unit(const Unit& u) {
    const std::size_t dk = u.dk, dv = u.dv, n = dv * dk, T = u.T;
    auto alpha_at = [&](std::size_t t) { return u.log_gate ? std::exp(u.gate[t * u.gs]) : u.gate[t * u.gs]; };
    auto resets = [&](std::size_t t) { return u.reset && (*u.reset)[t]; };

    // Forward once, keeping the state that enters every window.
    const std::size_t nwin = (T + kWindow - 1) / kWindow;
    std::vector<double> kept(nwin * n), S(n, 0.0), sk(dv), w(dv);
    if (u.init) std::copy(u.init, u.init + n, S.begin());
    for (std::size_t t = 0; t < T; ++t) {
        if (t % kWindow == 0) std::copy(S.begin(), S.end(), kept.begin() + (t / kWindow) * n);
        if (resets(t)) std::fill(S.begin(), S.end(), 0.0);
        step(S.data(), u.k + t * u.ks, u.v + t * u.vs, alpha_at(t), u.beta[t * u.gs], dv, dk, sk.data());
    }

    // Reverse scan, one window at a time: re-run the window from its kept
    // state, storing the entering (E) and resulting (A) state of each position.
    std::vector<double> dS(n, 0.0), E(kWindow * n), A(kWindow * n);
    if (u.d_final) std::copy(u.d_final, u.d_final + n, dS.begin());
    for (std::size_t c = nwin; c-- > 0;) {
        const std::size_t t0 = c * kWindow, t1 = std::min(T, t0 + kWindow);
        std::copy(kept.begin() + c * n, kept.begin() + (c + 1) * n, S.begin());
        for (std::size_t t = t0; t < t1; ++t) {
            if (resets(t)) std::fill(S.begin(), S.end(), 0.0);
            std::copy(S.begin(), S.end(), E.begin() + (t - t0) * n);
            step(S.data(), u.k + t * u.ks, u.v + t * u.vs, alpha_at(t), u.beta[t * u.gs], dv, dk, sk.data());
            std::copy(S.begin(), S.end(), A.begin() + (t - t0) * n);
        }
        for (std::size_t t = t1; t-- > t0;) {
            const double* P = &E[(t - t0) * n];
            const double* Sa = &A[(t - t0) * n];
            const double *q = u.q + t * u.qs, *k = u.k + t * u.ks, *v = u.v + t * u.vs, *dO = u.d_o + t * u.os;
            const double a = alpha_at(t), b = u.beta[t * u.gs];
            double* dq = u.dq + t * u.qs;
            double* dkt = u.dk_ + t * u.ks;
            double* dvt = u.dv_ + t * u.vs;
            // o = S q
            for (std::size_t j = 0; j < dk; ++j) {
                double acc = 0.0;
                for (std::size_t i = 0; i < dv; ++i) acc += Sa[i * dk + j] * dO[i];
                dq[j] = acc;
            }
            for (std::size_t i = 0; i < dv; ++i)
                for (std::size_t j = 0; j < dk; ++j) dS[i * dk + j] += dO[i] * q[j];
            // S = alpha (P - beta sk k^T) + beta v k^T
            double dalpha = 0.0, dbeta = 0.0;
            for (std::size_t i = 0; i < dv; ++i) {
                double s = 0.0, ww = 0.0;
                for (std::size_t j = 0; j < dk; ++j) {
                    s += P[i * dk + j] * k[j];
                    ww += dS[i * dk + j] * k[j];
                    dalpha += dS[i * dk + j] * P[i * dk + j];
                }
                sk[i] = s;
                w[i] = ww;
            }
            for (std::size_t i = 0; i < dv; ++i) {
                dalpha -= b * sk[i] * w[i];
                dbeta += (v[i] - a * sk[i]) * w[i];
                dvt[i] = b * w[i];
            }
            for (std::size_t j = 0; j < dk; ++j) {
                double acc = 0.0;
                for (std::size_t i = 0; i < dv; ++i)
                    acc += dS[i * dk + j] * (b * v[i] - a * b * sk[i]) - a * b * P[i * dk + j] * w[i];
                dkt[j] = acc;
            }
            u.dgate[t * u.gs] = u.log_gate ? dalpha * a : dalpha;
            u.dbeta[t * u.gs] = dbeta;
            if (resets(t)) {
                std::fill(dS.begin(), dS.end(), 0.0);  // the state before a reset does not reach S
            } else {
                for (std::size_t i = 0; i < dv; ++i)
                    for (std::size_t j = 0; j < dk; ++j) dS[i * dk + j] = a * (dS[i * dk + j] - b * w[i] * k[j]);
            }
        }
    }
    if (u.dinit) std::copy(dS.begin(), dS.end(), u.dinit);
}

}  // namespace

DeltaGrads gated_delta_sequential_backward(const DeltaInputs& inp, const DeltaState& init,
                                           const std::vector<double>& d_out, const DeltaState* d_final) {
    const std::size_t d = inp.head_dim, T = inp.len();
    require(d > 0, "gated_delta_sequential_backward: head_dim must be > 0");
    require(inp.q.size() >= T * d && inp.k.size() >= T * d && inp.v.size() >= T * d,
            "gated_delta_sequential_backward: q, k or v holds fewer than T x head_dim values");
    require(inp.beta.size() >= T && inp.segment.size() >= T,
            "gated_delta_sequential_backward: beta or segment is shorter than alpha");
    require(d_out.size() >= T * d, "gated_delta_sequential_backward: d_out holds fewer than T x head_dim values");
    require(init.s.size() == d * d, "gated_delta_sequential_backward: init is not head_dim x head_dim");
    require(!d_final || d_final->s.size() == d * d, "gated_delta_sequential_backward: d_final is not head_dim x head_dim");

    // delta.rs:139-143: a reset at t = 0 and at every segment change.
    std::vector<char> reset(T, 0);
    for (std::size_t t = 0; t < T; ++t) reset[t] = t == 0 || inp.segment[t] != inp.segment[t - 1];

    DeltaGrads g;
    g.q.assign(T * d, 0.0);
    g.k.assign(T * d, 0.0);
    g.v.assign(T * d, 0.0);
    g.alpha.assign(T, 0.0);
    g.beta.assign(T, 0.0);
    g.init = DeltaState::zeros(d);
    Unit u;
    u.T = T;
    u.dk = u.dv = d;
    u.q = inp.q.data();
    u.k = inp.k.data();
    u.v = inp.v.data();
    u.gate = inp.alpha.data();
    u.beta = inp.beta.data();
    u.d_o = d_out.data();
    u.qs = u.ks = u.vs = u.os = d;
    u.gs = 1;
    u.reset = &reset;
    u.init = init.s.data();
    u.d_final = d_final ? d_final->s.data() : nullptr;
    u.dq = g.q.data();
    u.dk_ = g.k.data();
    u.dv_ = g.v.data();
    u.dgate = g.alpha.data();
    u.dbeta = g.beta.data();
    u.dinit = g.init.s.data();
    backward_unit(u);
    return g;
}

void gated_delta_prefill_backward(const PrefillBackwardArgs& a) {
    require(a.batch >= 1 && a.heads >= 1 && a.d_k >= 1 && a.d_v >= 1 && a.seq_len >= 0,
            "gated_delta_prefill_backward: batch, heads, d_k, d_v must be >= 1 and seq_len >= 0");
    require(a.gate_kind == RHZ_GATE_LOG_ALPHA || a.gate_kind == RHZ_GATE_ALPHA,
            "gated_delta_prefill_backward: unknown gate_kind");
    const std::size_t H = a.heads, dk = a.d_k, dv = a.d_v, N = a.batch;
    const std::size_t tokens = a.cu_seqlens ? std::size_t(a.seq_len) : N * std::size_t(a.seq_len);
    if (a.cu_seqlens) {
        require(a.cu_seqlens[0] == 0 && a.cu_seqlens[N] == a.seq_len,
                "gated_delta_prefill_backward: cu_seqlens must run from 0 to seq_len");
        for (std::size_t s = 0; s < N; ++s)
            require(a.cu_seqlens[s + 1] >= a.cu_seqlens[s], "gated_delta_prefill_backward: cu_seqlens must be non-decreasing");
    }
    if (tokens > 0)
        require(a.q && a.k && a.v && a.gate && a.beta && a.d_o && a.dq && a.dk && a.dv && a.dgate && a.dbeta,
                "gated_delta_prefill_backward: an input or gradient pointer is NULL");

    const std::size_t units = N * H;
    std::atomic<std::size_t> next{0};
    auto worker = [&] {
        for (std::size_t i = next++; i < units; i = next++) {
            const std::size_t s = i / H, h = i % H;
            const std::size_t t0 = a.cu_seqlens ? std::size_t(a.cu_seqlens[s]) : s * std::size_t(a.seq_len);
            const std::size_t t1 = a.cu_seqlens ? std::size_t(a.cu_seqlens[s + 1]) : t0 + std::size_t(a.seq_len);
            Unit u;
            u.T = t1 - t0;
            u.dk = dk;
            u.dv = dv;
            u.qs = u.ks = H * dk;
            u.vs = u.os = H * dv;
            u.gs = H;
            const std::size_t r = t0 * H + h;
            u.q = a.q + r * dk;
            u.k = a.k + r * dk;
            u.v = a.v + r * dv;
            u.gate = a.gate + r;
            u.beta = a.beta + r;
            u.d_o = a.d_o + r * dv;
            u.log_gate = a.gate_kind == RHZ_GATE_LOG_ALPHA;
            u.init = a.initial_state ? a.initial_state + i * dv * dk : nullptr;
            u.d_final = a.d_final_state ? a.d_final_state + i * dv * dk : nullptr;
            u.dq = a.dq + r * dk;
            u.dk_ = a.dk + r * dk;
            u.dv_ = a.dv + r * dv;
            u.dgate = a.dgate + r;
            u.dbeta = a.dbeta + r;
            u.dinit = a.d_initial_state ? a.d_initial_state + i * dv * dk : nullptr;
            backward_unit(u);
        }
    };
    const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
    const std::size_t nthreads = std::min<std::size_t>(units, a.threads > 0 ? std::size_t(a.threads) : hw);
    if (nthreads <= 1) {
        worker();
        return;
    }
    std::vector<std::thread> pool;
    for (std::size_t i = 0; i < nthreads; ++i) pool.emplace_back(worker);
    for (auto& t : pool) t.join();
}

namespace gradcheck {

double central_difference(const std::function<double(const std::vector<double>&)>& f, const std::vector<double>& x,
                          std::size_t i) {
    const double h = 1e-5;
    std::vector<double> xp = x, xm = x;
    xp[i] += h;
    xm[i] -= h;
    return (f(xp) - f(xm)) / (2.0 * h);
}

GradCheckReport check(const std::function<double(const std::vector<double>&)>& f, const std::vector<double>& x,
                      const std::vector<double>& analytic) {
    GradCheckReport r;
    for (std::size_t i = 0; i < x.size(); ++i) {
        const double fd = central_difference(f, x, i);
        const double denom = std::max({std::fabs(fd), std::fabs(analytic[i]), 1e-6});
        const double rel = std::fabs(fd - analytic[i]) / denom;
        if (rel > r.max_rel_err) {
            r.max_rel_err = rel;
            r.worst_index = i;
        }
    }
    return r;
}

}  // namespace gradcheck
}  // namespace ops
}  // namespace rhizome
