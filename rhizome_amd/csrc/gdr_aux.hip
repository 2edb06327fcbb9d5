// gdr_aux.hip -- the Local-block steps on either side of the gated delta-rule
// (SPEC.md:53-63), for gfx950.  All three are HBM-bound: each reads its
// inputs once and writes its outputs once.
//
//   conv1d_kernel    causal depthwise conv1d of width 4 with a carried
//                    3-sample state (causal_conv1d_step, delta.rs:232-243),
//                    batched over packed sequences and channels;
//   prepare_kernel   q, k L2-normalised (q rescaled), beta = sigmoid(logit),
//                    g = -softplus(a_h) softplus(logit) (elementwise.rs:5-12,
//                    36-42, 125-128);
//   conv_prepare_kernel  the two above in one pass over the [q | k | v]
//                    projections (SPEC.md:53-56);
//   rmsnorm_kernel   RMSNorm of rows with a learned scale (norm.rs:8-13),
//                    the per-head norm of the op's output (norm.rs:48-59).

#include <type_traits>

#include "gdr_device.hpp"
#include "gdr_internal.hpp"

namespace rhz {
namespace {

// N consecutive elements as floats: one 16-byte access when VEC (N = 4 fp32
// or 8 bf16, 16-byte aligned), else N = 1.
template <typename T, bool VEC>
struct Vec {
    static constexpr int N = VEC ? 16 / int(sizeof(T)) : 1;
    // the loaded bits, unpacked later (4 registers for 16 bytes)
    using Raw = typename std::conditional<VEC, uint4, T>::type;
    static __device__ __forceinline__ Raw load_raw(const T* p) { return *reinterpret_cast<const Raw*>(p); }
    static __device__ __forceinline__ void unpack(const Raw& r, float (&x)[N]) {
        if constexpr (!VEC) {
            x[0] = Elem<T>::load(&r, 0);
        } else if constexpr (sizeof(T) == 4) {
            x[0] = __uint_as_float(r.x); x[1] = __uint_as_float(r.y);
            x[2] = __uint_as_float(r.z); x[3] = __uint_as_float(r.w);
        } else {
            const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                x[2 * i] = __uint_as_float(w[i] << 16);
                x[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
            }
        }
    }
    static __device__ __forceinline__ void load(const T* p, float (&x)[N]) { unpack(load_raw(p), x); }
    // NT: a non-temporal store (streaming output that this kernel does not
    // read back).
    template <bool NT = false>
    static __device__ __forceinline__ void store(T* p, const float (&x)[N]) {
        if constexpr (!VEC) {
            Elem<T>::store(p, 0, x[0]);
        } else if constexpr (sizeof(T) == 4) {
            const f32x4 v = {x[0], x[1], x[2], x[3]};
            if constexpr (NT)
                __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(p));
            else
                *reinterpret_cast<f32x4*>(p) = v;
        } else {
            typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
            const u32x4 u = {pack_bf16x2(x[0], x[1]), pack_bf16x2(x[2], x[3]), pack_bf16x2(x[4], x[5]),
                             pack_bf16x2(x[6], x[7])};
            if constexpr (NT)
                __builtin_nontemporal_store(u, reinterpret_cast<u32x4*>(p));
            else
                *reinterpret_cast<u32x4*>(p) = u;
        }
    }
};

__host__ __device__ inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ---------------------------------------------------------------- conv1d
// Thread = (channel, span of kConvSpan consecutive tokens of the pack); a
// span may cross sequence starts.  Each thread rebuilds its window of the
// three previous inputs from x (or the sequence's initial state before its
// start), so spans are independent and the grid covers tokens x channels.
constexpr int kConvSpan = 16;
// conv_prepare: spans of 16 tokens, and register use bounded for three
// waves per SIMD (measured 74.4 against 80.0 us at two waves per SIMD, on
// 16384 tokens x 6144 bf16 channels).
constexpr int kConvPrepSpan = 16;
constexpr int kConvPrepWaves = 3;
constexpr bool kConvNT = true;  // y by non-temporal stores
constexpr bool kRowNT = true;   // prepare's and RMSNorm's outputs by non-temporal stores

struct ConvParams {
    const void* x;
    const float* w;
    const float* bias;
    const int* cu;
    const float* init;
    float* fin;
    void* y;
    int batch, seq_len, C;
};

// Sequence containing token t (packed: last s with cu[s] <= t; offsets are
// clamped into [0, total]).
__device__ __forceinline__ int seq_of(const ConvParams& p, int t) {
    if (!p.cu) return t / max(p.seq_len, 1);
    int lo = 0, hi = p.batch - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (min(max(p.cu[mid], 0), p.seq_len) <= t) lo = mid; else hi = mid - 1;
    }
    return lo;
}
__device__ __forceinline__ int seq_start(const ConvParams& p, int s) {
    return p.cu ? min(max(p.cu[s], 0), p.seq_len) : s * p.seq_len;
}
__device__ __forceinline__ int seq_end(const ConvParams& p, int s) {
    if (!p.cu) return (s + 1) * p.seq_len;
    return min(max(p.cu[s + 1], seq_start(p, s)), p.seq_len);
}

// Grid: one dimension, block b = (span b / ncb, channel block b % ncb);
// each thread owns N consecutive channels (one 16-byte access per token
// when VEC).  The span's outputs go to emit(t, c, y[N]), called for every
// token of the span that lies in a sequence, in token order, by every thread
// of the block at once (the tokens are the block's, so the calls stay
// converged across the block).
template <typename T, bool VEC, int SPAN, typename Emit>
__device__ __forceinline__ void conv_span(const ConvParams& p, int total, int ncb, Emit&& emit) {
    using V = Vec<T, VEC>;
    constexpr int N = V::N;
    const int c = ((blockIdx.x % ncb) * 256 + threadIdx.x) * N;
    const int t0 = (blockIdx.x / ncb) * SPAN;
    if (c >= p.C || t0 >= total) return;
    const int t1 = min(t0 + SPAN, total);
    const T* __restrict__ x = static_cast<const T*>(p.x);  // the outputs never overlap x
    const long C = p.C;
    float w[N][4], b[N];
    if (aligned16(p.w)) {  // uniform: one 16-byte load per channel
#pragma unroll
        for (int e = 0; e < N; ++e) {
            const float4 f = reinterpret_cast<const float4*>(p.w)[c + e];
            w[e][0] = f.x;
            w[e][1] = f.y;
            w[e][2] = f.z;
            w[e][3] = f.w;
        }
    } else {
#pragma unroll
        for (int e = 0; e < N; ++e)
#pragma unroll
            for (int j = 0; j < 4; ++j) w[e][j] = p.w[4 * (c + e) + j];
    }
#pragma unroll
    for (int e = 0; e < N; ++e) b[e] = p.bias ? p.bias[c + e] : 0.f;

    int s = seq_of(p, t0);
    int s0 = seq_start(p, s), s1 = seq_end(p, s);
    if (t1 - t0 == SPAN && t0 - 3 >= s0 && t1 <= s1) {
        // A whole span inside one sequence, three tokens or more past its
        // start: the window comes from x and no state is reset or read, so
        // the span is straight-line code with every load issued up front.
        float a[3][N];
        typename V::Raw ws[3], xs[SPAN];
#pragma unroll
        for (int j = 0; j < 3; ++j) ws[j] = V::load_raw(x + (t0 - 3 + j) * C + c);
#pragma unroll
        for (int i = 0; i < SPAN; ++i) xs[i] = V::load_raw(x + (t0 + i) * C + c);
#pragma unroll
        for (int j = 0; j < 3; ++j) V::unpack(ws[j], a[j]);
#pragma unroll
        for (int i = 0; i < SPAN; ++i) {
            float xt[N], yt[N];
            V::unpack(xs[i], xt);
#pragma unroll
            for (int e = 0; e < N; ++e)  // delta.rs:237-238, evaluated left to right
                yt[e] = w[e][0] * a[0][e] + w[e][1] * a[1][e] + w[e][2] * a[2][e] + w[e][3] * xt[e] + b[e];
            emit(t0 + i, c, yt);
#pragma unroll
            for (int e = 0; e < N; ++e) {
                a[0][e] = a[1][e];
                a[1][e] = a[2][e];
                a[2][e] = xt[e];
            }
        }
        if (t1 == s1 && p.fin) {
#pragma unroll
            for (int e = 0; e < N; ++e) {
                float* f = p.fin + ((long)s * C + c + e) * 3;
                f[0] = a[0][e];
                f[1] = a[1][e];
                f[2] = a[2][e];
            }
        }
        return;
    }
    // a[j][e]: input at position t - 3 + j of channel c + e (oldest first);
    // before a sequence start the values come from its state, or are zero
    float a[3][N];
    auto window = [&](int seq, int start, int pos, float (&dst)[N]) {
        if (pos >= start) {
            V::load(x + pos * C + c, dst);
        } else {
            const int k = 3 + (pos - start);  // 0..2
#pragma unroll
            for (int e = 0; e < N; ++e) dst[e] = p.init ? p.init[((long)seq * C + c + e) * 3 + k] : 0.f;
        }
    };
#pragma unroll
    for (int j = 0; j < 3; ++j) window(s, s0, t0 - 3 + j, a[j]);
    // every input of the span first, so that its loads overlap
    typename V::Raw xs[SPAN];
#pragma unroll
    for (int i = 0; i < SPAN; ++i)
        if (t0 + i < t1) xs[i] = V::load_raw(x + (t0 + i) * C + c);
#pragma unroll
    for (int i = 0; i < SPAN; ++i) {
        const int t = t0 + i;
        if (t >= t1) break;
        while (t >= s1) {  // next sequence (skipping empty ones)
            if (s + 1 >= p.batch) return;  // past the last sequence: not part of any
            ++s;
            s0 = seq_start(p, s);
            s1 = seq_end(p, s);
#pragma unroll
            for (int j = 0; j < 3; ++j) window(s, s0, s0 - 3 + j, a[j]);
        }
        float xt[N], yt[N];
        V::unpack(xs[i], xt);
#pragma unroll
        for (int e = 0; e < N; ++e)  // delta.rs:237-238, evaluated left to right
            yt[e] = w[e][0] * a[0][e] + w[e][1] * a[1][e] + w[e][2] * a[2][e] + w[e][3] * xt[e] + b[e];
        emit(t, c, yt);
#pragma unroll
        for (int e = 0; e < N; ++e) {
            a[0][e] = a[1][e];
            a[1][e] = a[2][e];
            a[2][e] = xt[e];
        }
        if (t == s1 - 1 && p.fin) {
#pragma unroll
            for (int e = 0; e < N; ++e) {
                float* f = p.fin + ((long)s * C + c + e) * 3;
                f[0] = a[0][e];
                f[1] = a[1][e];
                f[2] = a[2][e];
            }
        }
    }
}

template <typename T, bool VEC>
__global__ __launch_bounds__(256) void conv1d_kernel(ConvParams p, int total, int ncb) {
    using V = Vec<T, VEC>;
    T* __restrict__ y = static_cast<T*>(p.y);
    const long C = p.C;
    conv_span<T, VEC, kConvSpan>(p, total, ncb, [&](int t, int c, const float (&yt)[V::N]) {
        V::template store<kConvNT>(y + t * C + c, yt);
    });
}

// ------------------------------------------------------- conv1d + prepare
// The Local block's prologue in one pass: causal conv1d over x = [q | k | v]
// projections (C = H (2 d_k + d_v) channels per token), then prepare's maps
// on the convolved values before they are rounded -- q rows l2-normalised
// and scaled, k rows l2-normalised (elementwise.rs:125-128), v passed on --
// written as separate q [tokens, H, d_k], k [tokens, H, d_k], v [tokens, H,
// d_v], with beta = sigmoid(beta_logit) and g = -softplus(a_log[h])
// softplus(alpha_logit) per (token, head) (elementwise.rs:5-12, 36-42).  A
// q or k row is G = d_k / N consecutive threads of a block (channel blocks
// are whole rows), so its sum of squares is a sum over those lanes.
struct ConvPrepParams {
    ConvParams conv;
    void* q;
    void* k;
    void* v;
    const float* beta_logit;
    const float* alpha_logit;
    const float* a_log;
    float* beta;
    float* g;
    int heads, d_k, d_v;
    float q_scale;
};

template <int G>
__device__ __forceinline__ float row_sum(float x) {
    if constexpr (G >= 32) {
        x = lane_group_sum<16>(x);
        x += __shfl_xor(x, 16, kWave);
        if constexpr (G == 64) x += __shfl_xor(x, 32, kWave);
        return x;
    } else if constexpr (G > 1) {
        return lane_group_sum<G>(x);
    } else {
        return x;
    }
}

template <typename T, int G>
__global__ __launch_bounds__(256, kConvPrepWaves) void conv_prepare_kernel(ConvPrepParams p, int total, int ncb) {
    using V = Vec<T, true>;
    constexpr int N = V::N;
    const int H = p.heads, dk = p.d_k, dv = p.d_v;
    const int qk = H * dk;  // channels of q (and of k)
    T* __restrict__ qo = static_cast<T*>(p.q);
    T* __restrict__ ko = static_cast<T*>(p.k);
    T* __restrict__ vo = static_cast<T*>(p.v);
    conv_span<T, true, kConvPrepSpan>(p.conv, total, ncb, [&](int t, int c, const float (&yt)[N]) {
        if (c >= 2 * qk) {  // v (uniform over the row's lanes)
            V::template store<kConvNT>(vo + (long)t * H * dv + (c - 2 * qk), yt);
            return;
        }
        const bool isq = c < qk;
        const int cc = isq ? c : c - qk;  // channel within q or k
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < N; ++e) ss += yt[e] * yt[e];
        ss = row_sum<G>(ss);
        // x / max(||x||, 1e-12) * scale (elementwise.rs:126-127), the
        // reciprocal norm as v_rsq_f32 of max(||x||^2, 1e-24) (about 1 ulp)
        const float f = (isq ? p.q_scale : 1.f) * __builtin_amdgcn_rsqf(fmaxf(ss, 1e-24f));
        float o[N];
#pragma unroll
        for (int e = 0; e < N; ++e) o[e] = yt[e] * f;
        V::template store<kRowNT>((isq ? qo : ko) + (long)t * qk + cc, o);
    });
    // The gates of the block's (token, head) pairs, one pair per thread: the
    // blocks holding q channels cover every head once per span.
    const int cb = (blockIdx.x % ncb) * 256 * N;  // first channel of the block
    const int t0 = (blockIdx.x / ncb) * kConvPrepSpan;
    if (cb >= qk || t0 >= total) return;
    const int h0 = cb / dk, nh = (min(cb + 256 * N, qk) - cb) / dk;
    const int nt = min(t0 + kConvPrepSpan, total) - t0;
    for (int i = threadIdx.x; i < nt * nh; i += 256) {
        const int h = h0 + i % nh;
        const long r = (long)(t0 + i / nh) * H + h;
        p.beta[r] = sigmoid_f(p.beta_logit[r]);
        p.g[r] = -softplus_f(p.a_log[h]) * softplus_f(p.alpha_logit[r]);
    }
}

// Final state of every empty sequence: its initial state (or zeros).
// Grid: channel blocks x sequences (grid-stride over sequences).
__global__ __launch_bounds__(256) void conv1d_empty_kernel(ConvParams p) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c >= p.C) return;
    for (int s = blockIdx.y; s < p.batch; s += gridDim.y) {
        if (seq_end(p, s) > seq_start(p, s)) continue;
        const long o = ((long)s * p.C + c) * 3;
#pragma unroll
        for (int k = 0; k < 3; ++k) p.fin[o + k] = p.init ? p.init[o + k] : 0.f;
    }
}

// ---------------------------------------------------------------- prepare
// A group of G lanes per (token, head) row; lane li holds elements li + G i.
struct PrepParams {
    const void* q_in;
    const void* k_in;
    void* q_out;
    void* k_out;
    const float* beta_logit;
    const float* alpha_logit;
    const float* a_log;
    float* beta;
    float* g;
    int rows, heads, d;
    float q_scale;
};


// A row of d elements as vectors of N: lane li of the row's G lanes holds
// vectors li + G i, i < NV (zero beyond the row).
template <int G, int NV, typename T, bool VEC>
struct RowSlice {
    using V = Vec<T, VEC>;
    static constexpr int N = V::N;
    float v[NV][N];
    typename V::Raw raw[NV];
    // issue() starts the loads, reduce() unpacks them and returns the row's
    // sum of squares; rows whose loads are all issued first overlap them.
    __device__ __forceinline__ void issue(const T* row, int d, int li) {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int j = (li + G * i) * N;
            if (j < d) raw[i] = V::load_raw(row + j);
        }
    }
    __device__ __forceinline__ float reduce(int d, int li) {
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int j = (li + G * i) * N;
            if (j < d) {
                V::unpack(raw[i], v[i]);
            } else {
#pragma unroll
                for (int e = 0; e < N; ++e) v[i][e] = 0.f;
            }
#pragma unroll
            for (int e = 0; e < N; ++e) ss += v[i][e] * v[i][e];
        }
        return group_sum<G>(ss);
    }
    __device__ __forceinline__ float load(const T* row, int d, int li) {
        issue(row, d, li);
        return reduce(d, li);
    }
    template <typename F>
    __device__ __forceinline__ void store(T* row, int d, int li, F f) {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int j = (li + G * i) * N;
            if (j < d) {
                float o[N];
#pragma unroll
                for (int e = 0; e < N; ++e) o[e] = f(j + e, v[i][e]);
                V::template store<kRowNT>(row + j, o);
            }
        }
    }
};

// q and k of a (token, head) row L2-normalised (elementwise.rs:126-127: x /
// max(|x|, 1e-12) * scale), and its gates.  Every load of the row is issued
// before the first store, which also makes q_out = q_in and k_out = k_in safe.
// A group of G lanes handles rows r and r + RPB of its block's 2 RPB rows.
template <int G, int NV, typename T, bool VEC>
__global__ __launch_bounds__(256) void prepare_kernel(PrepParams p) {
    constexpr int RPB = 256 / G;
    const int row0 = blockIdx.x * 2 * RPB + threadIdx.x / G;
    const int li = threadIdx.x % G;
    RowSlice<G, NV, T, VEC> rq[2], rk[2];
    float bl[2] = {0.f, 0.f}, al[2] = {0.f, 0.f}, ah[2] = {0.f, 0.f};
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int row = row0 + u * RPB;
        if (row >= p.rows) break;  // uniform over the group (G divides 64)
        const long base = (long)row * p.d;
        rq[u].issue(static_cast<const T*>(p.q_in) + base, p.d, li);
        rk[u].issue(static_cast<const T*>(p.k_in) + base, p.d, li);
        if (li == 0) {
            bl[u] = p.beta_logit[row];
            al[u] = p.alpha_logit[row];
            ah[u] = p.a_log[row % p.heads];
        }
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int row = row0 + u * RPB;
        if (row >= p.rows) break;
        const long base = (long)row * p.d;
        const float fq = p.q_scale / fmaxf(sqrtf(rq[u].reduce(p.d, li)), 1e-12f);
        const float fk = 1.f / fmaxf(sqrtf(rk[u].reduce(p.d, li)), 1e-12f);
        rq[u].store(static_cast<T*>(p.q_out) + base, p.d, li, [&](int, float x) { return x * fq; });
        rk[u].store(static_cast<T*>(p.k_out) + base, p.d, li, [&](int, float x) { return x * fk; });
        if (li == 0) {
            p.beta[row] = sigmoid_f(bl[u]);
            p.g[row] = -softplus_f(ah[u]) * softplus_f(al[u]);
        }
    }
}

// ---------------------------------------------------------------- rmsnorm
struct NormParams {
    const void* x;
    const float* scale;
    void* y;
    int rows, dim;
    float eps;
};

// A group of G lanes handles rows r and r + RPB of its block's 2 RPB rows.
template <int G, int NV, typename T, bool VEC>
__global__ __launch_bounds__(256) void rmsnorm_kernel(NormParams p) {
    constexpr int RPB = 256 / G;
    const int row0 = blockIdx.x * 2 * RPB + threadIdx.x / G;
    const int li = threadIdx.x % G;
    RowSlice<G, NV, T, VEC> r[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int row = row0 + u * RPB;
        if (row >= p.rows) break;  // uniform over the group
        r[u].issue(static_cast<const T*>(p.x) + (long)row * p.dim, p.dim, li);
    }
    const float* scale = p.scale;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int row = row0 + u * RPB;
        if (row >= p.rows) break;
        const float inv = 1.f / sqrtf(r[u].reduce(p.dim, li) / (float)p.dim + p.eps);  // norm.rs:9-11
        r[u].store(static_cast<T*>(p.y) + (long)row * p.dim, p.dim, li,
                   [&](int j, float x) { return x * inv * scale[j]; });
    }
}

// Rows of n elements: G lanes per row, NV vectors of N per lane (G NV N >= n).
template <template <int, int, typename, bool> class K, int G, int NV, typename T, bool VEC, typename P>
hipError_t go_rows(const P& p, int rows, hipStream_t st) {
    constexpr int RPB = 256 / G;  // rows per block and pass; each block takes two passes
    hipLaunchKernelGGL((K<G, NV, T, VEC>::fn), dim3((rows + 2 * RPB - 1) / (2 * RPB)), dim3(256), 0, st, p);
    return hipGetLastError();
}
template <int G, int NV, typename T, bool VEC>
struct PrepK {
    static constexpr auto fn = prepare_kernel<G, NV, T, VEC>;
};
template <int G, int NV, typename T, bool VEC>
struct NormK {
    static constexpr auto fn = rmsnorm_kernel<G, NV, T, VEC>;
};
// Vectors of 16 bytes when every row starts 16-byte aligned; the lanes per
// row then cover n / N vectors.  PAIR: rows of 9..16 vectors on 8 lanes with
// two vectors each (prepare, d_k = 128 bf16: 5.95 against 5.57 TB/s with 16
// lanes of one vector; RMSNorm of the same rows measured 6.04 against 6.27,
// and 4 lanes of four vectors 5.35 and 5.27).
template <template <int, int, typename, bool> class K, typename T, bool PAIR = false, typename P>
hipError_t pick_rows(const P& p, int rows, int n, bool vec, hipStream_t st) {
    if (rows <= 0) return hipSuccess;
    if (vec) {
        const int nv = n / (16 / int(sizeof(T)));  // vectors per row
        if (nv <= 8) return go_rows<K, 8, 1, T, true>(p, rows, st);
        if (nv <= 16) {
            if constexpr (PAIR) return go_rows<K, 8, 2, T, true>(p, rows, st);
            return go_rows<K, 16, 1, T, true>(p, rows, st);
        }
        if (nv <= 32) return go_rows<K, 32, 1, T, true>(p, rows, st);
        if (nv <= 64) return go_rows<K, 64, 1, T, true>(p, rows, st);
        if (nv <= 128) return go_rows<K, 64, 2, T, true>(p, rows, st);
        return go_rows<K, 64, 4, T, true>(p, rows, st);  // n <= 1024 elements of 4 bytes
    }
    if (n <= 64) return go_rows<K, 16, 4, T, false>(p, rows, st);
    if (n <= 128) return go_rows<K, 32, 4, T, false>(p, rows, st);
    if (n <= 256) return go_rows<K, 32, 8, T, false>(p, rows, st);
    if (n <= 512) return go_rows<K, 64, 8, T, false>(p, rows, st);
    return go_rows<K, 64, 16, T, false>(p, rows, st);
}

}  // namespace

hipError_t launch_conv1d(const rhz_conv1d_args& a, hipStream_t st) {
    ConvParams p{a.x, a.weight, a.bias, a.cu_seqlens, a.initial_state, a.final_state, a.y,
                 a.batch, a.seq_len, a.channels};
    const int total = a.cu_seqlens ? a.seq_len : a.batch * a.seq_len;
    const int es = a.dtype == RHZ_F32 ? 4 : 2, nvec = 16 / es;
    const bool vec = a.channels % nvec == 0 && aligned16(a.x) && aligned16(a.y);
    const int per_thread = vec ? nvec : 1;
    const int ncb = (a.channels / per_thread + 255) / 256;
    if (total > 0) {
        const dim3 grid((unsigned)((long)ncb * ((total + kConvSpan - 1) / kConvSpan)));
        if (a.dtype == RHZ_F32) {
            if (vec) hipLaunchKernelGGL((conv1d_kernel<float, true>), grid, dim3(256), 0, st, p, total, ncb);
            else hipLaunchKernelGGL((conv1d_kernel<float, false>), grid, dim3(256), 0, st, p, total, ncb);
        } else {
            if (vec) hipLaunchKernelGGL((conv1d_kernel<uint16_t, true>), grid, dim3(256), 0, st, p, total, ncb);
            else hipLaunchKernelGGL((conv1d_kernel<uint16_t, false>), grid, dim3(256), 0, st, p, total, ncb);
        }
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    if (a.final_state) {
        // one channel per thread, whatever the main kernel's vector width
        const int ecb = (a.channels + 255) / 256;
        hipLaunchKernelGGL(conv1d_empty_kernel, dim3(ecb, min(a.batch, 65535)), dim3(256), 0, st, p);
        return hipGetLastError();
    }
    return hipSuccess;
}

bool conv_prepare_supported(int dtype, int d_k, int d_v) {
    const int n = dtype == RHZ_F32 ? 4 : 8;  // elements per 16-byte access
    if (d_k % n != 0 || d_v % n != 0) return false;
    const int g = d_k / n;
    return g == 1 || g == 2 || g == 4 || g == 8 || g == 16 || g == 32 || g == 64;
}

hipError_t launch_conv_prepare(const rhz_gdr_conv_prepare_args& a, hipStream_t st) {
    const int C = a.heads * (2 * a.d_k + a.d_v);
    ConvPrepParams p{{a.x, a.weight, a.bias, a.cu_seqlens, a.initial_state, a.final_state, nullptr, a.batch,
                      a.seq_len, C},
                     a.q, a.k, a.v, a.beta_logit, a.alpha_logit, a.a_log, a.beta, a.g,
                     a.heads, a.d_k, a.d_v, a.q_scale};
    const int total = a.cu_seqlens ? a.seq_len : a.batch * a.seq_len;
    const int n = a.dtype == RHZ_F32 ? 4 : 8;
    const int g = a.d_k / n;
    const int ncb = (C / n + 255) / 256;
    if (total > 0) {
        const dim3 grid((unsigned)((long)ncb * ((total + kConvPrepSpan - 1) / kConvPrepSpan)));
#define RHZ_CONV_PREP(T, G) hipLaunchKernelGGL((conv_prepare_kernel<T, G>), grid, dim3(256), 0, st, p, total, ncb)
        if (a.dtype == RHZ_F32) {
            switch (g) {
                case 1: RHZ_CONV_PREP(float, 1); break;
                case 2: RHZ_CONV_PREP(float, 2); break;
                case 4: RHZ_CONV_PREP(float, 4); break;
                case 8: RHZ_CONV_PREP(float, 8); break;
                case 16: RHZ_CONV_PREP(float, 16); break;
                case 32: RHZ_CONV_PREP(float, 32); break;
                default: RHZ_CONV_PREP(float, 64); break;
            }
        } else {
            switch (g) {
                case 1: RHZ_CONV_PREP(uint16_t, 1); break;
                case 2: RHZ_CONV_PREP(uint16_t, 2); break;
                case 4: RHZ_CONV_PREP(uint16_t, 4); break;
                case 8: RHZ_CONV_PREP(uint16_t, 8); break;
                case 16: RHZ_CONV_PREP(uint16_t, 16); break;
                case 32: RHZ_CONV_PREP(uint16_t, 32); break;
                default: RHZ_CONV_PREP(uint16_t, 64); break;
            }
        }
#undef RHZ_CONV_PREP
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    if (a.final_state) {
        const int ecb = (C + 255) / 256;
        hipLaunchKernelGGL(conv1d_empty_kernel, dim3(ecb, min(a.batch, 65535)), dim3(256), 0, st, p.conv);
        return hipGetLastError();
    }
    return hipSuccess;
}

hipError_t launch_prepare(const rhz_gdr_prepare_args& a, hipStream_t st) {
    PrepParams p{a.q_in, a.k_in, a.q_out, a.k_out, a.beta_logit, a.alpha_logit, a.a_log, a.beta, a.g,
                 a.tokens * a.heads, a.heads, a.d_k, a.q_scale};
    const int nvec = a.dtype == RHZ_F32 ? 4 : 8;
    const bool vec = a.d_k % nvec == 0 && aligned16(a.q_in) && aligned16(a.k_in) && aligned16(a.q_out) &&
                     aligned16(a.k_out);
    if (a.dtype == RHZ_F32) return pick_rows<PrepK, float, true>(p, p.rows, a.d_k, vec, st);
    return pick_rows<PrepK, uint16_t, true>(p, p.rows, a.d_k, vec, st);
}

hipError_t launch_rmsnorm(const rhz_rmsnorm_args& a, hipStream_t st) {
    NormParams p{a.x, a.scale, a.y, a.rows, a.dim, a.eps};
    const int nvec = a.dtype == RHZ_F32 ? 4 : 8;
    const bool vec = a.dim % nvec == 0 && aligned16(a.x) && aligned16(a.y);
    if (a.dtype == RHZ_F32) return pick_rows<NormK, float>(p, a.rows, a.dim, vec, st);
    return pick_rows<NormK, uint16_t>(p, a.rows, a.dim, vec, st);
}

}  // namespace rhz
