/*
 * gdr_oracle.c -- CPU f64 oracle for the gated delta-rule (GDR) forward.
 *
 * TEST INFRASTRUCTURE ONLY.  It is the reference that tests compare against, never the product:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * it.  The shipped library (rhizome_amd/librhizome_gdr.so) never links,
 * calls or falls back to anything here.
 *
 * It restates, loop for loop, the f64 reference of RHIZOME's `crates/ops`:
 *
 *   orc_gated_delta_step        crates/ops/src/delta.rs:94-127
 *   orc_gated_delta_sequential  crates/ops/src/delta.rs:133-154
 *   orc_gated_delta_scan_chunked crates/ops/src/delta.rs:159-197
 *   orc_gated_delta_multistep   crates/ops/src/delta.rs:202-230
 *   orc_causal_conv1d_step      crates/ops/src/delta.rs:236-243
 *   orc_conv1d_batched          the same step along packed sequences and channels
 *   orc_rmsnorm_rows            crates/ops/src/norm.rs:8-13 (and 48-59 per head)
 *   orc_make_inputs             crates/ops/src/delta.rs:254-280 (test fixture builder)
 *   Philox-4x32-10              crates/ops/src/rng.rs:7-90
 *   orc_sigmoid / orc_softplus / orc_l2norm
 *                               crates/ops/src/elementwise.rs:5-12, 36-42, 125-128
 *
 * The recurrence uses only f64 +, -, * in the reference's evaluation order.
 * Built with -ffp-contract=off (no FMA contraction, as in Rust) the results
 * are the IEEE-754 results of the reference itself.
 *
 * Extensions beyond the reference API (each pinned by a property test, not
 * by the reference, which has no such function):
 *   orc_gdr_steps_rect     -- the step loop WITHOUT the t=0 reset and with a
 *                             rectangular d_v x d_k state (rows of S are
 *                             independent, so a d_v split equals the joint
 *                             run exactly; tests pin this against the square
 *                             reference).
 *   orc_gdr_prefill_batched / orc_gdr_decode_batched -- the same step loop
 *                             over packed [tokens, heads, dim] buffers,
 *                             OpenMP-parallel over independent (seq, head).
 *
 * Pins (tests/test_oracle.py): Random123 Philox known-answer vectors; the
 * seven delta.rs unit tests; closed forms (beta=0 pure decay, one-hot
 * overwrite, d=1 scalar recurrence, linearity in v and q, row independence,
 * chunk-size invariance, segment reset, alpha=0 reset, non-expansiveness);
 * brute-force dense-matrix evaluation of the recurrence on tiny inputs.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ */
/* Philox-4x32-10: crates/ops/src/rng.rs:7-10 (constants), 43-60 (block) */
/* ------------------------------------------------------------------ */
#define ORC_W0 0x9E3779B9u
#define ORC_W1 0xBB67AE85u
#define ORC_M0 0xD2511F53u
#define ORC_M1 0xCD9E8D57u

/* rng.rs:43-60: counter words [ctr_lo, ctr_hi, stream_lo, stream_hi],
 * key (seed_hi, seed_lo), ten rounds, key bumped after every round. */
void orc_philox_block(uint64_t seed, uint64_t stream, uint64_t counter, uint32_t out[4])
{
    uint32_t c0 = (uint32_t)counter, c1 = (uint32_t)(counter >> 32);
    uint32_t c2 = (uint32_t)stream, c3 = (uint32_t)(stream >> 32);
    uint32_t k0 = (uint32_t)(seed >> 32), k1 = (uint32_t)seed;
    for (int r = 0; r < 10; ++r) {
        uint64_t p0 = (uint64_t)c0 * ORC_M0;
        uint64_t p1 = (uint64_t)c2 * ORC_M1;
        uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
        uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
        uint32_t n0 = hi1 ^ c1 ^ k0, n1 = lo1, n2 = hi0 ^ c3 ^ k1, n3 = lo0;
        c0 = n0; c1 = n1; c2 = n2; c3 = n3;
        k0 += ORC_W0;
        k1 += ORC_W1;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

typedef struct {
    uint64_t seed, stream, counter;
    uint32_t buf[4];
    int cursor;
} orc_philox;

/* rng.rs:25-33 */
static void ph_init(orc_philox* p, uint64_t seed, uint64_t stream)
{
    p->seed = seed;
    p->stream = stream;
    p->counter = 0;
    p->cursor = 4;
}

/* rng.rs:63-72 */
static uint32_t ph_next_u32(orc_philox* p)
{
    if (p->cursor >= 4) {
        orc_philox_block(p->seed, p->stream, p->counter, p->buf);
        p->counter += 1;
        p->cursor = 0;
    }
    return p->buf[p->cursor++];
}

/* rng.rs:78-82: 27 high bits then 26 low bits, / 2^53 */
static double ph_next_f64(orc_philox* p)
{
    uint64_t hi = (uint64_t)(ph_next_u32(p) >> 5);
    uint64_t lo = (uint64_t)(ph_next_u32(p) >> 6);
    return (double)((hi << 26) | lo) / (double)(1ull << 53);
}

/* core::f64::consts::TAU, the correctly rounded double of 2*pi */
#define ORC_TAU 6.28318530717958647692528676655900577

/* rng.rs:85-90: Box-Muller, cosine branch, u1 floored at 1e-300 */
static double ph_next_normal(orc_philox* p)
{
    double u1 = ph_next_f64(p);
    if (u1 < 1e-300) u1 = 1e-300;
    double u2 = ph_next_f64(p);
    return sqrt(-2.0 * log(u1)) * cos(ORC_TAU * u2);
}

void orc_philox_u32(uint64_t seed, uint64_t stream, int64_t n, uint32_t* out)
{
    orc_philox p;
    ph_init(&p, seed, stream);
    for (int64_t i = 0; i < n; ++i) out[i] = ph_next_u32(&p);
}

void orc_philox_f64(uint64_t seed, uint64_t stream, int64_t n, double* out)
{
    orc_philox p;
    ph_init(&p, seed, stream);
    for (int64_t i = 0; i < n; ++i) out[i] = ph_next_f64(&p);
}

/* n normals of stream (seed, stream) scaled as mean + std * z.  Normal #i
 * consumes exactly one Philox block (four words), so the i-th normal is a
 * pure function of block(i); the loop is parallel over i for speed and
 * gives the same values as the sequential generator. */
void orc_philox_normal(uint64_t seed, uint64_t stream, int64_t n, double mean, double std_,
                       double* out, int nthreads)
{
#ifdef _OPENMP
    if (nthreads < 1) nthreads = 1;
#pragma omp parallel for schedule(static) num_threads(nthreads)
#endif
    for (int64_t i = 0; i < n; ++i) {
        orc_philox p;
        ph_init(&p, seed, stream);
        p.counter = (uint64_t)i;
        double z = ph_next_normal(&p);
        out[i] = (mean == 0.0 && std_ == 1.0) ? z : mean + std_ * z;
    }
}

/* ------------------------------------------------------------------ */
/* Elementwise: crates/ops/src/elementwise.rs                          */
/* ------------------------------------------------------------------ */

/* elementwise.rs:5-12 */
double orc_sigmoid(double x)
{
    if (x >= 0.0) return 1.0 / (1.0 + exp(-x));
    double e = exp(x);
    return e / (1.0 + e);
}

/* elementwise.rs:36-42 (linear above 30) */
double orc_softplus(double x)
{
    if (x > 30.0) return x;
    return log(1.0 + exp(x));
}

/* elementwise.rs:125-128: n = sqrt(sum v^2).max(1e-12); v / n * scale */
void orc_l2norm(const double* x, int64_t n, double scale, double* out)
{
    double s = 0.0;
    for (int64_t i = 0; i < n; ++i) s += x[i] * x[i];
    double nrm = sqrt(s);
    if (nrm < 1e-12) nrm = 1e-12;
    for (int64_t i = 0; i < n; ++i) out[i] = x[i] / nrm * scale;
}

void orc_l2norm_rows(double* x, int64_t rows, int64_t d, double scale, int nthreads)
{
#ifdef _OPENMP
    if (nthreads < 1) nthreads = 1;
#pragma omp parallel for schedule(static) num_threads(nthreads)
#endif
    for (int64_t r = 0; r < rows; ++r) orc_l2norm(x + r * d, d, scale, x + r * d);
}

void orc_sigmoid_vec(const double* z, int64_t n, double* out)
{
    for (int64_t i = 0; i < n; ++i) out[i] = orc_sigmoid(z[i]);
}

void orc_neg_softplus_vec(const double* z, int64_t n, double* out)
{
    for (int64_t i = 0; i < n; ++i) out[i] = -orc_softplus(z[i]);
}

void orc_exp_vec(const double* z, int64_t n, double* out)
{
    for (int64_t i = 0; i < n; ++i) out[i] = exp(z[i]);
}

/* ------------------------------------------------------------------ */
/* Gated delta rule: crates/ops/src/delta.rs                           */
/* ------------------------------------------------------------------ */

/* One position on a d_v x d_k state S[i][j] at i*d_k + j (i = value row,
 * j = key column), the three passes of delta.rs:104-125 in their order and
 * with their parenthesisation.  With d_k == d_v == d this is
 * gated_delta_step itself. */
static void step_rect(double* s, int64_t dk, int64_t dv, const double* q, const double* k,
                      const double* v, double alpha, double beta, double* sk, double* o)
{
    for (int64_t i = 0; i < dv; ++i) { /* delta.rs:105-111 */
        double acc = 0.0;
        for (int64_t j = 0; j < dk; ++j) acc += s[i * dk + j] * k[j];
        sk[i] = acc;
    }
    for (int64_t i = 0; i < dv; ++i) { /* delta.rs:112-117 */
        for (int64_t j = 0; j < dk; ++j) {
            double decayed = alpha * (s[i * dk + j] - beta * sk[i] * k[j]);
            s[i * dk + j] = decayed + beta * v[i] * k[j];
        }
    }
    for (int64_t i = 0; i < dv; ++i) { /* delta.rs:118-125 */
        double acc = 0.0;
        for (int64_t j = 0; j < dk; ++j) acc += s[i * dk + j] * q[j];
        o[i] = acc;
    }
}

/* delta.rs:94-127.  Like the reference, each call allocates its two
 * d-vectors (sk, o) and hands o back to the caller, who frees it. */
double* orc_gated_delta_step(double* s, int64_t d, const double* q, const double* k,
                             const double* v, double alpha, double beta)
{
    double* sk = (double*)calloc((size_t)d, sizeof(double));
    double* o = (double*)calloc((size_t)d, sizeof(double));
    step_rect(s, d, d, q, k, v, alpha, beta, sk, o);
    free(sk);
    return o;
}

void orc_free(void* p) { free(p); }

/* delta.rs:133-154.  NOTE the reference quirk: prev_segment starts as None,
 * so the state is reset at t = 0 and `init` never reaches the output. */
void orc_gated_delta_sequential(int64_t t_len, int64_t d, const double* q, const double* k,
                                const double* v, const double* alpha, const double* beta,
                                const uint64_t* segment, const double* init, double* out,
                                double* final_state)
{
    int64_t dd = d * d;
    double* state = (double*)malloc((size_t)(dd > 0 ? dd : 1) * sizeof(double));
    memcpy(state, init, (size_t)dd * sizeof(double));
    int have_prev = 0;
    uint64_t prev = 0;
    for (int64_t t = 0; t < t_len; ++t) {
        if (!have_prev || prev != segment[t]) {
            memset(state, 0, (size_t)dd * sizeof(double));
            prev = segment[t];
            have_prev = 1;
        }
        double* o = orc_gated_delta_step(state, d, q + t * d, k + t * d, v + t * d, alpha[t],
                                         beta[t]);
        memcpy(out + t * d, o, (size_t)d * sizeof(double));
        free(o);
    }
    memcpy(final_state, state, (size_t)dd * sizeof(double));
    free(state);
}

/* delta.rs:159-197: chunks clipped at segment changes, reset when
 * start == 0 or the segment changes; the chunk size never changes the
 * arithmetic (the reference calls the same step per position). */
void orc_gated_delta_scan_chunked(int64_t t_len, int64_t d, const double* q, const double* k,
                                  const double* v, const double* alpha, const double* beta,
                                  const uint64_t* segment, const double* init, int64_t chunk,
                                  double* out, double* final_state)
{
    if (chunk < 1) chunk = 1;
    int64_t dd = d * d;
    double* state = (double*)malloc((size_t)(dd > 0 ? dd : 1) * sizeof(double));
    memcpy(state, init, (size_t)dd * sizeof(double));
    memset(out, 0, (size_t)(t_len * d) * sizeof(double));
    int64_t start = 0;
    while (start < t_len) {
        int64_t end = start + chunk < t_len ? start + chunk : t_len;
        for (int64_t t = start + 1; t < end; ++t) {
            if (segment[t] != segment[start]) {
                end = t;
                break;
            }
        }
        if (start == 0 || segment[start] != segment[start - 1])
            memset(state, 0, (size_t)dd * sizeof(double));
        for (int64_t t = start; t < end; ++t) {
            double* o = orc_gated_delta_step(state, d, q + t * d, k + t * d, v + t * d,
                                             alpha[t], beta[t]);
            memcpy(out + t * d, o, (size_t)d * sizeof(double));
            free(o);
        }
        start = end;
    }
    memcpy(final_state, state, (size_t)dd * sizeof(double));
    free(state);
}

/* delta.rs:202-230: n = min(T, max_positions) positions, the state after
 * every position is returned ([n][d*d]); same reset-at-t=0 quirk. */
int64_t orc_gated_delta_multistep(int64_t t_len, int64_t d, const double* q, const double* k,
                                  const double* v, const double* alpha, const double* beta,
                                  const uint64_t* segment, const double* init,
                                  int64_t max_positions, double* outs, double* states)
{
    int64_t n = t_len < max_positions ? t_len : max_positions;
    int64_t dd = d * d;
    double* state = (double*)malloc((size_t)(dd > 0 ? dd : 1) * sizeof(double));
    memcpy(state, init, (size_t)dd * sizeof(double));
    int have_prev = 0;
    uint64_t prev = 0;
    for (int64_t t = 0; t < n; ++t) {
        if (!have_prev || prev != segment[t]) {
            memset(state, 0, (size_t)dd * sizeof(double));
            prev = segment[t];
            have_prev = 1;
        }
        double* o = orc_gated_delta_step(state, d, q + t * d, k + t * d, v + t * d, alpha[t],
                                         beta[t]);
        memcpy(outs + t * d, o, (size_t)d * sizeof(double));
        free(o);
        memcpy(states + t * dd, state, (size_t)dd * sizeof(double));
    }
    free(state);
    return n;
}

/* delta.rs:236-243 */
double orc_causal_conv1d_step(double state[3], const double weight[4], double x, double bias)
{
    double y = weight[0] * state[0] + weight[1] * state[1] + weight[2] * state[2] +
               weight[3] * x + bias;
    state[0] = state[1];
    state[1] = state[2];
    state[2] = x;
    return y;
}

/* causal_conv1d_step (delta.rs:236-243) along every sequence of a pack and
 * every channel: x [tokens, C], weight [C][4], bias [C] or NULL, state
 * [n][C][3] from init (or zeros) at each sequence start, final state into
 * fin (may be NULL).  Tokens outside every sequence are not written. */
void orc_conv1d_batched(int64_t n_seqs, const int64_t* cu_seqlens, int64_t C, const double* x,
                        const double* weight, const double* bias, const double* init, double* y,
                        double* fin)
{
    for (int64_t s = 0; s < n_seqs; ++s) {
        for (int64_t c = 0; c < C; ++c) {
            double st[3] = {0.0, 0.0, 0.0};
            if (init) memcpy(st, init + (s * C + c) * 3, sizeof st);
            for (int64_t t = cu_seqlens[s]; t < cu_seqlens[s + 1]; ++t)
                y[t * C + c] = orc_causal_conv1d_step(st, weight + 4 * c, x[t * C + c], bias ? bias[c] : 0.0);
            if (fin) memcpy(fin + (s * C + c) * 3, st, sizeof st);
        }
    }
}

/* norm.rs:8-13 on every row of `dim` values (groupnorm_heads, norm.rs:48-59,
 * is this on each head's slice). */
void orc_rmsnorm_rows(int64_t rows, int64_t dim, const double* x, const double* scale, double eps, double* y)
{
    for (int64_t r = 0; r < rows; ++r) {
        const double* xr = x + r * dim;
        double ss = 0.0;
        for (int64_t i = 0; i < dim; ++i) ss += xr[i] * xr[i];
        double ms = ss / (double)dim;
        double inv = 1.0 / sqrt(ms + eps);
        for (int64_t i = 0; i < dim; ++i) y[r * dim + i] = xr[i] * inv * scale[i];
    }
}

/* delta.rs:254-280 (the reference's test-fixture builder): stream 17 gives
 * q (L2-normalised rows scaled by sqrt(d), floor 1e-9) then k (scale 1);
 * stream 18 gives v, then alpha = 0.5 + 0.5u, then beta = 0.1 + 0.8u. */
void orc_make_inputs(int64_t t_len, int64_t d, uint64_t seed, double* q, double* k, double* v,
                     double* alpha, double* beta)
{
    orc_philox r;
    ph_init(&r, seed, 17);
    double* rows[2] = {q, k};
    double scales[2] = {sqrt((double)d), 1.0};
    for (int which = 0; which < 2; ++which) {
        double* dst = rows[which];
        for (int64_t t = 0; t < t_len; ++t) {
            double* row = dst + t * d;
            double ss = 0.0;
            for (int64_t j = 0; j < d; ++j) row[j] = ph_next_normal(&r);
            for (int64_t j = 0; j < d; ++j) ss += row[j] * row[j];
            double nrm = sqrt(ss);
            if (nrm < 1e-9) nrm = 1e-9;
            for (int64_t j = 0; j < d; ++j) row[j] = row[j] / nrm * scales[which];
        }
    }
    orc_philox r2;
    ph_init(&r2, seed, 18);
    for (int64_t i = 0; i < t_len * d; ++i) v[i] = ph_next_normal(&r2);
    for (int64_t t = 0; t < t_len; ++t) alpha[t] = 0.5 + 0.5 * ph_next_f64(&r2);
    for (int64_t t = 0; t < t_len; ++t) beta[t] = 0.1 + 0.8 * ph_next_f64(&r2);
}

/* ------------------------------------------------------------------ */
/* Extensions over the reference API (see the file header)             */
/* ------------------------------------------------------------------ */

/* The step loop of delta.rs:138-152 without the t=0 reset, on a d_v x d_k
 * state: state is taken as given and updated in place.  q/k/v rows are at
 * stride q_stride/k_stride/v_stride, outputs at o_stride, gates at g_stride. */
void orc_gdr_steps_rect(int64_t t_len, int64_t dk, int64_t dv, const double* q, int64_t q_stride,
                        const double* k, int64_t k_stride, const double* v, int64_t v_stride,
                        const double* alpha, const double* beta, int64_t g_stride, double* state,
                        double* o, int64_t o_stride)
{
    double* sk = (double*)malloc((size_t)(dv > 0 ? dv : 1) * sizeof(double));
    for (int64_t t = 0; t < t_len; ++t)
        step_rect(state, dk, dv, q + t * q_stride, k + t * k_stride, v + t * v_stride,
                  alpha[t * g_stride], beta[t * g_stride], sk, o + t * o_stride);
    free(sk);
}

/* Packed prefill: q,k [tokens][H][dk], v,o [tokens][H][dv], alpha,beta
 * [tokens][H], init/final [n_seqs][H][dv][dk] (init NULL = zeros, final
 * NULL = not returned).  cu_seqlens[n_seqs+1] int64.  Each (seq, head) is
 * an independent step loop, run in parallel with nthreads threads. */
void orc_gdr_prefill_batched(int64_t n_seqs, const int64_t* cu_seqlens, int64_t heads,
                             int64_t dk, int64_t dv, const double* q, const double* k,
                             const double* v, const double* alpha, const double* beta,
                             const double* init, double* o, double* final_state, int nthreads)
{
    int64_t units = n_seqs * heads;
#ifdef _OPENMP
    if (nthreads < 1) nthreads = 1;
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads)
#endif
    for (int64_t u = 0; u < units; ++u) {
        int64_t n = u / heads, h = u % heads;
        int64_t t0 = cu_seqlens[n], t1 = cu_seqlens[n + 1];
        double* st = (double*)malloc((size_t)(dv * dk) * sizeof(double));
        if (init)
            memcpy(st, init + u * dv * dk, (size_t)(dv * dk) * sizeof(double));
        else
            memset(st, 0, (size_t)(dv * dk) * sizeof(double));
        if (t1 > t0)
            orc_gdr_steps_rect(t1 - t0, dk, dv, q + (t0 * heads + h) * dk, heads * dk,
                               k + (t0 * heads + h) * dk, heads * dk, v + (t0 * heads + h) * dv,
                               heads * dv, alpha + t0 * heads + h, beta + t0 * heads + h, heads,
                               st, o + (t0 * heads + h) * dv, heads * dv);
        if (final_state) memcpy(final_state + u * dv * dk, st, (size_t)(dv * dk) * sizeof(double));
        free(st);
    }
}

/* One decode step for every (b, h): q,k [B][H][dk], v,o [B][H][dv],
 * alpha,beta [B][H], state [B][H][dv][dk] updated in place. */
void orc_gdr_decode_batched(int64_t batch, int64_t heads, int64_t dk, int64_t dv, const double* q,
                            const double* k, const double* v, const double* alpha,
                            const double* beta, double* state, double* o, int nthreads)
{
    int64_t units = batch * heads;
#ifdef _OPENMP
    if (nthreads < 1) nthreads = 1;
#pragma omp parallel for schedule(static) num_threads(nthreads)
#endif
    for (int64_t u = 0; u < units; ++u)
        orc_gdr_steps_rect(1, dk, dv, q + u * dk, dk, k + u * dk, dk, v + u * dv, dv, alpha + u,
                           beta + u, 1, state + u * dv * dk, o + u * dv, dv);
}

int orc_max_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ------------------------------------------------------------------ */
/* CPU baseline timing (bench.py cpu_baseline leg)                     */
/* ------------------------------------------------------------------ */

/* gated_delta_sequential (delta.rs:133-154, with its per-step allocations)
 * over n_units independent heads stored unit-major ([unit][T][d] for q, k,
 * v; [unit][T] for alpha, beta), nthreads-way parallel over units.  Outputs
 * go to out [unit][T][d] and final [unit][d][d]. */
void orc_bench_sequential(int64_t n_units, int64_t t_len, int64_t d, const double* q,
                          const double* k, const double* v, const double* alpha,
                          const double* beta, double* out, double* final_state, int nthreads)
{
#ifdef _OPENMP
    if (nthreads < 1) nthreads = 1;
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads)
#endif
    for (int64_t u = 0; u < n_units; ++u) {
        uint64_t* seg = (uint64_t*)calloc((size_t)(t_len > 0 ? t_len : 1), sizeof(uint64_t));
        double* init = (double*)calloc((size_t)(d * d), sizeof(double));
        orc_gated_delta_sequential(t_len, d, q + u * t_len * d, k + u * t_len * d,
                                   v + u * t_len * d, alpha + u * t_len, beta + u * t_len, seg,
                                   init, out + u * t_len * d, final_state + u * d * d);
        free(init);
        free(seg);
    }
}

/* gated_delta_step (delta.rs:94-127) once for each of n_units heads:
 * q, k, v [unit][d], alpha, beta [unit], state [unit][d][d] in place. */
void orc_bench_step(int64_t n_units, int64_t d, const double* q, const double* k, const double* v,
                    const double* alpha, const double* beta, double* state, double* o,
                    int nthreads)
{
#ifdef _OPENMP
    if (nthreads < 1) nthreads = 1;
#pragma omp parallel for schedule(static) num_threads(nthreads)
#endif
    for (int64_t u = 0; u < n_units; ++u) {
        double* r = orc_gated_delta_step(state + u * d * d, d, q + u * d, k + u * d, v + u * d,
                                         alpha[u], beta[u]);
        memcpy(o + u * d, r, (size_t)d * sizeof(double));
        free(r);
    }
}
