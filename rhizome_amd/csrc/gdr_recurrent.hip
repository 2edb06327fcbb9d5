// gdr_recurrent.hip -- row-parallel fp32 gated delta-rule kernels for gfx950:
//
//   gdr_decode_kernel     one position for every (b, h), state streamed from
//                         HBM and written back in place (gated_delta_step,
//                         crates/ops/src/delta.rs:94-127, batched);
//   gdr_multistep_kernel  up to a few positions for every (b, h) with the
//                         state rows in registers, writing o and the state
//                         after every position (gated_delta_multistep,
//                         delta.rs:202-230, batched, without its t = 0 reset);
//   gdr_staged_recurrent_kernel, gdr_recurrent_kernel
//                         the same update carried token by token through a
//                         whole sequence with the state rows in registers
//                         (gated_delta_sequential, delta.rs:133-154, without
//                         its t = 0 reset; the fp32-input prefill path), with
//                         the positions staged through LDS in blocks (d_k <=
//                         128) or loaded one position ahead (any shape).
//
// Rows of S are independent (row i only reads v_i and its own row), so
// both kernels give each row to a group of LPR = d_k_max / 16 lanes; lane li
// of a group holds columns c*4*LPR + 4*li + e (c, e in 0..3), so every
// 16-byte load of a wave covers whole contiguous row segments.  Per row and
// token the two dot products S_i.k and S_i.q and the shared k.q are summed
// over the group with a fixed butterfly, then
//     c_i  = beta * (v_i - alpha * (S_i.k))
//     o_i  = alpha * (S_i.q) + c_i * (k.q)        (= S_i' . q)
//     S_i' = alpha * S_i + c_i * k                (one FMA per element)
// so the state is read once and written once per position.

#include "gdr_device.hpp"
#include "gdr_internal.hpp"

namespace rhz {
namespace {

struct StepParams {
    const void* q;
    const void* k;
    const void* v;
    const float* gate;
    const float* beta;
    float* state;
    void* o;
    int d_k, d_v, gate_is_alpha;
};

struct MultiParams {
    const void* q;
    const void* k;
    const void* v;
    const float* gate;
    const float* beta;
    const float* state;
    float* states;
    void* o;
    int steps, heads, d_k, d_v, gate_is_alpha;
};

struct SeqParams {
    const void* q;
    const void* k;
    const void* v;
    const float* gate;
    const float* beta;
    const int* cu_seqlens;
    const float* init;
    float* fin;
    void* o;
    int seq_len, heads, d_k, d_v, gate_is_alpha;
};

// The 16 columns of a row held by lane li of its group (zero outside [0, n)).
template <int LPR, bool VEC, typename T>
__device__ __forceinline__ void load_slice(const T* row, int li, int n, float (&x)[16]) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int col = c * 4 * LPR + 4 * li;
        if (VEC) {
            float4 f = make_float4(0.f, 0.f, 0.f, 0.f);
            if (col < n) f = load4(row + col);
            x[4 * c + 0] = f.x;
            x[4 * c + 1] = f.y;
            x[4 * c + 2] = f.z;
            x[4 * c + 3] = f.w;
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) x[4 * c + e] = (col + e < n) ? Elem<T>::load(row, col + e) : 0.f;
        }
    }
}

// The same rows by non-temporal loads (a state streamed through once).
template <int LPR>
__device__ __forceinline__ void load_slice_nt(const float* row, int li, int n, float (&x)[16]) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int col = c * 4 * LPR + 4 * li;
        f32x4 f = {0.f, 0.f, 0.f, 0.f};
        if (col < n) f = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(row + col));
        x[4 * c + 0] = f[0];
        x[4 * c + 1] = f[1];
        x[4 * c + 2] = f[2];
        x[4 * c + 3] = f[3];
    }
}

// NT: non-temporal stores (streaming output that this kernel does not read
// back, such as the multistep snapshots).
template <int LPR, bool VEC, bool NT = false>
__device__ __forceinline__ void store_slice(float* row, int li, int n, const float (&x)[16]) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int col = c * 4 * LPR + 4 * li;
        if (VEC) {
            if (col < n) {
                if (NT) {
                    const f32x4 val = {x[4 * c + 0], x[4 * c + 1], x[4 * c + 2], x[4 * c + 3]};
                    __builtin_nontemporal_store(val, reinterpret_cast<f32x4*>(row + col));
                } else {
                    *reinterpret_cast<float4*>(row + col) =
                        make_float4(x[4 * c + 0], x[4 * c + 1], x[4 * c + 2], x[4 * c + 3]);
                }
            }
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (col + e < n) row[col + e] = x[4 * c + e];
        }
    }
}

__device__ __forceinline__ float dot16(const float (&a)[16], const float (&b)[16]) {
    float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        s0 += a[4 * c + 0] * b[4 * c + 0];
        s1 += a[4 * c + 1] * b[4 * c + 1];
        s2 += a[4 * c + 2] * b[4 * c + 2];
        s3 += a[4 * c + 3] * b[4 * c + 3];
    }
    return (s0 + s1) + (s2 + s3);
}

// Sequence bounds of packed sequence `seq`, clamped into [0, total].
__device__ __forceinline__ void seq_bounds(const int* cu, int seq, int seq_len, int& t0, int& t1) {
    if (cu) {
        t0 = min(max(cu[seq], 0), seq_len);
        t1 = min(max(cu[seq + 1], t0), seq_len);
    } else {
        t0 = seq * seq_len;
        t1 = t0 + seq_len;
    }
}

// ---------------------------------------------------------------- decode
// Grid: x = b*H + h, y = block of P*RPP rows.  256 threads, RPP = 256/LPR
// rows per pass; all of a lane's state loads are issued before any use.
// NTL: the state is read by non-temporal loads (states well past the
// last-level cache, chosen by the launch).
template <int LPR, int P, bool VEC, typename T, bool NTL = false>
__global__ __launch_bounds__(256) void gdr_decode_kernel(StepParams p) {
    constexpr int RPP = 256 / LPR;
    const int bh = blockIdx.x;
    const int li = threadIdx.x % LPR;
    const int rl = threadIdx.x / LPR;
    const int dk = p.d_k, dv = p.d_v;
    const T* q = static_cast<const T*>(p.q) + (long)bh * dk;
    const T* k = static_cast<const T*>(p.k) + (long)bh * dk;
    const T* v = static_cast<const T*>(p.v) + (long)bh * dv;
    T* o = static_cast<T*>(p.o) + (long)bh * dv;
    float* S = p.state + (long)bh * dv * dk;
    const int rbase = blockIdx.y * (P * RPP) + rl;

    float s[P][16];
#pragma unroll
    for (int pp = 0; pp < P; ++pp) {
        const int r = rbase + pp * RPP;
        if (r < dv) {
            if constexpr (NTL && VEC)
                load_slice_nt<LPR>(S + (long)r * dk, li, dk, s[pp]);
            else
                load_slice<LPR, VEC, float>(S + (long)r * dk, li, dk, s[pp]);
        } else {
#pragma unroll
            for (int e = 0; e < 16; ++e) s[pp][e] = 0.f;
        }
    }
    float kr[16], qr[16];
    load_slice<LPR, VEC, T>(k, li, dk, kr);
    load_slice<LPR, VEC, T>(q, li, dk, qr);
    const float alpha = decay_factor(p.gate[bh], p.gate_is_alpha);
    const float beta = p.beta[bh];
    const float kq = group_sum<LPR>(dot16(kr, qr));

#pragma unroll
    for (int pp = 0; pp < P; ++pp) {
        const int r = rbase + pp * RPP;
        const float sk = group_sum<LPR>(dot16(s[pp], kr));
        const float sq = group_sum<LPR>(dot16(s[pp], qr));
        if (r < dv) {
            // Contractions written out, so that every instance (P, NTL)
            // rounds alike and the streamed and plain launches agree bit
            // for bit.
            const float vi = Elem<T>::load(v, r);
            const float c = beta * fmaf(-alpha, sk, vi);
            const float oi = fmaf(alpha, sq, c * kq);
#pragma unroll
            for (int e = 0; e < 16; ++e) s[pp][e] = fmaf(alpha, s[pp][e], c * kr[e]);
            store_slice<LPR, VEC, true>(S + (long)r * dk, li, dk, s[pp]);
            if (li == 0) Elem<T>::store(o, r, oi);
        }
    }
}

// ------------------------------------------------------------- multistep
// Grid: x = b*H + h, y = block of P*RPP rows, as the decode kernel; the rows
// stay in registers across the n positions.  Each position's k, q, v and
// gates are loaded when it starts: without a second register set for the
// next position the kernel needs 92 VGPRs instead of 125, and the fifth wave
// per SIMD this allows hides the load latency better than prefetching did
// (473.7 vs 480.1 us at B = 256, H = 16, d = 128, 8 positions).
template <int LPR, int P, bool VEC, typename T>
__global__ __launch_bounds__(256) void gdr_multistep_kernel(MultiParams p) {
    constexpr int RPP = 256 / LPR;
    const int bh = blockIdx.x;
    const int b = bh / p.heads, h = bh - b * p.heads;
    const int li = threadIdx.x % LPR;
    const int rl = threadIdx.x / LPR;
    const int dk = p.d_k, dv = p.d_v, H = p.heads, n = p.steps;
    const int rbase = blockIdx.y * (P * RPP) + rl;
    const float* S0 = p.state + (long)bh * dv * dk;

    float s[P][16];
#pragma unroll
    for (int pp = 0; pp < P; ++pp) {
        const int r = rbase + pp * RPP;
        if (r < dv) {
            load_slice<LPR, VEC, float>(S0 + (long)r * dk, li, dk, s[pp]);
        } else {
#pragma unroll
            for (int e = 0; e < 16; ++e) s[pp][e] = 0.f;
        }
    }
    const T* qp = static_cast<const T*>(p.q);
    const T* kp = static_cast<const T*>(p.k);
    const T* vp = static_cast<const T*>(p.v);
    T* op = static_cast<T*>(p.o);

    // position t of (b, h): row (b n + t) H + h of every [B, n, H, ...] tensor
    float kn[16], qn[16], vn[P], gn = 0.f, bn = 0.f;
    auto fetch = [&](int t) {
        const long th = ((long)b * n + t) * H + h;
        load_slice<LPR, VEC, T>(kp + th * dk, li, dk, kn);
        load_slice<LPR, VEC, T>(qp + th * dk, li, dk, qn);
#pragma unroll
        for (int pp = 0; pp < P; ++pp) {
            const int r = rbase + pp * RPP;
            vn[pp] = r < dv ? Elem<T>::load(vp, th * dv + r) : 0.f;
        }
        gn = p.gate[th];
        bn = p.beta[th];
    };
    for (int t = 0; t < n; ++t) {
        fetch(t);
        float kr[16], qr[16], vr[P];
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            kr[e] = kn[e];
            qr[e] = qn[e];
        }
#pragma unroll
        for (int pp = 0; pp < P; ++pp) vr[pp] = vn[pp];
        const float ga = gn, be = bn;
        const float alpha = decay_factor(ga, p.gate_is_alpha);
        const float kq = group_sum<LPR>(dot16(kr, qr));
        const long th = ((long)b * n + t) * H + h;
        float* snap = p.states + th * dv * dk;
#pragma unroll
        for (int pp = 0; pp < P; ++pp) {
            const int r = rbase + pp * RPP;
            const float sk = group_sum<LPR>(dot16(s[pp], kr));
            const float sq = group_sum<LPR>(dot16(s[pp], qr));
            const float c = be * fmaf(-alpha, sk, vr[pp]);
            const float oi = fmaf(alpha, sq, c * kq);
#pragma unroll
            for (int e = 0; e < 16; ++e) s[pp][e] = fmaf(alpha, s[pp][e], c * kr[e]);
            if (r < dv) {
                store_slice<LPR, VEC, true>(snap + (long)r * dk, li, dk, s[pp]);
                if (li == 0) Elem<T>::store(op, th * dv + r, oi);
            }
        }
    }
}

// ------------------------------------------------------- recurrent prefill
// Grid: x = seq*H + h, y = block of RPW = 64/LPR rows; one wave per block.
// The next token's k, q, v and gates are loaded while the current one is
// applied.
template <int LPR, bool VEC, typename T>
__global__ __launch_bounds__(64) void gdr_recurrent_kernel(SeqParams p) {
    constexpr int RPW = 64 / LPR;
    const int unit = blockIdx.x;
    const int seq = unit / p.heads, h = unit % p.heads;
    const int li = threadIdx.x % LPR;
    const int r = blockIdx.y * RPW + threadIdx.x / LPR;
    const int dk = p.d_k, dv = p.d_v, H = p.heads;
    const bool row_ok = r < dv;
    int t0, t1;
    seq_bounds(p.cu_seqlens, seq, p.seq_len, t0, t1);

    float s[16];
    if (p.init && row_ok) {
        load_slice<LPR, VEC, float>(p.init + ((long)unit * dv + r) * dk, li, dk, s);
    } else {
#pragma unroll
        for (int e = 0; e < 16; ++e) s[e] = 0.f;
    }
    const T* qp = static_cast<const T*>(p.q);
    const T* kp = static_cast<const T*>(p.k);
    const T* vp = static_cast<const T*>(p.v);
    T* op = static_cast<T*>(p.o);

    float kn[16], qn[16], vn = 0.f, gn = 0.f, bn = 0.f;
    auto fetch = [&](int t) {
        const long th = (long)t * H + h;
        load_slice<LPR, VEC, T>(kp + th * dk, li, dk, kn);
        load_slice<LPR, VEC, T>(qp + th * dk, li, dk, qn);
        vn = row_ok ? Elem<T>::load(vp, th * dv + r) : 0.f;
        gn = p.gate[th];
        bn = p.beta[th];
    };
    if (t0 < t1) fetch(t0);
    for (int t = t0; t < t1; ++t) {
        float kr[16], qr[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            kr[e] = kn[e];
            qr[e] = qn[e];
        }
        const float vi = vn, ga = gn, be = bn;
        if (t + 1 < t1) fetch(t + 1);
        const float alpha = decay_factor(ga, p.gate_is_alpha);
        const float kq = group_sum<LPR>(dot16(kr, qr));
        const float sk = group_sum<LPR>(dot16(s, kr));
        const float sq = group_sum<LPR>(dot16(s, qr));
        const float c = be * fmaf(-alpha, sk, vi);
        const float oi = fmaf(alpha, sq, c * kq);
#pragma unroll
        for (int e = 0; e < 16; ++e) s[e] = fmaf(alpha, s[e], c * kr[e]);
        if (li == 0 && row_ok) Elem<T>::store(op, ((long)t * H + h) * dv + r, oi);
    }
    if (p.fin && row_ok) store_slice<LPR, VEC>(p.fin + ((long)unit * dv + r) * dk, li, dk, s);
}

// ------------------------------------------------ staged recurrent prefill
// The same recurrence with the positions staged through LDS in blocks of
// kStageTokens, for d_k <= 128 (LPR = 2, 4 or 8).  One workgroup of four
// waves per (sequence, head, 4 * 64 / LPR rows): every thread loads its
// share of block b + 1 -- k and q rows of the head, the workgroup's v rows,
// the gates -- into registers while the waves run block b from LDS, then
// writes it to the other LDS buffer together with k.q of each position
// (summed once per workgroup instead of once per row).  A wave then reads
// each position's k and q from LDS, sums S_i.k and S_i.q over its row's
// lanes by DPP, and updates its rows as gdr_recurrent_kernel does.  The
// global loads of a block have a whole block's compute to arrive.
constexpr int kStageTokens = 32;
constexpr int kStageWaves = 4;

template <int LPR>
struct StageSmem {
    static constexpr int DKP = 16 * LPR;                    // padded key width
    static constexpr int RPB = kStageWaves * (64 / LPR);    // state rows per workgroup
    float k[2][kStageTokens][DKP];
    float q[2][kStageTokens][DKP];
    float v[2][kStageTokens][RPB];
    float4 gb[2][kStageTokens];  // (alpha, beta, k.q, 0)
};

// One block's inputs in registers between their global load and their LDS
// write.  Piece m of thread j is float4 number f = j + 256 m of the block's
// row-major [token][DKP] k (and q) tile; v likewise over [token][RPB].
template <int LPR>
struct StageRegs {
    static constexpr int NKQ = kStageTokens * (16 * LPR) / 4 / 256;
    static constexpr int NV = kStageTokens * (kStageWaves * (64 / LPR)) / 4 / 256;
    float4 k[NKQ], q[NKQ], v[NV];
    float g, b;
};

template <int LPR, typename T>
__device__ __forceinline__ void stage_load(const SeqParams& p, int h, int i0, int tb, int len, int j,
                                           StageRegs<LPR>& r) {
    constexpr int DKP = 16 * LPR, RPB = kStageWaves * (64 / LPR);
    const long H = p.heads;
    const T* kp = static_cast<const T*>(p.k);
    const T* qp = static_cast<const T*>(p.q);
    const T* vp = static_cast<const T*>(p.v);
    const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int m = 0; m < StageRegs<LPR>::NKQ; ++m) {
        const int f = j + 256 * m, tt = f / (DKP / 4), col = 4 * (f % (DKP / 4));
        const bool ok = tt < len && col < p.d_k;
        const long off = ((long)(tb + tt) * H + h) * p.d_k + col;
        r.k[m] = ok ? load4(kp + off) : z;
        r.q[m] = ok ? load4(qp + off) : z;
    }
#pragma unroll
    for (int m = 0; m < StageRegs<LPR>::NV; ++m) {
        const int f = j + 256 * m, tt = f / (RPB / 4), rr = 4 * (f % (RPB / 4));
        const bool ok = tt < len && i0 + rr < p.d_v;
        r.v[m] = ok ? load4(vp + ((long)(tb + tt) * H + h) * p.d_v + i0 + rr) : z;
    }
    const int tt = j & (kStageTokens - 1);
    const bool ok = j < 2 * kStageTokens && tt < len;
    const float x = ok ? (j < kStageTokens ? p.gate : p.beta)[(long)(tb + tt) * H + h] : 0.f;
    r.g = x;  // lanes 0..31: gates, 32..63: betas (consumed by wave 0)
    r.b = x;
}

// Writes a block from registers to LDS buffer B, with alpha, beta and k.q of
// every position.  Positions past the sequence's end hold zeros.
template <int LPR>
__device__ __forceinline__ void stage_store(const SeqParams& p, StageSmem<LPR>& sm, int B, int j,
                                            const StageRegs<LPR>& r) {
    constexpr int DKP = 16 * LPR, RPB = kStageWaves * (64 / LPR);
    constexpr int PPT = DKP / 4;  // float4 pieces per position: a group of PPT consecutive threads
#pragma unroll
    for (int m = 0; m < StageRegs<LPR>::NKQ; ++m) {
        const int f = j + 256 * m, tt = f / PPT, col = 4 * (f % PPT);
        *reinterpret_cast<float4*>(&sm.k[B][tt][col]) = r.k[m];
        *reinterpret_cast<float4*>(&sm.q[B][tt][col]) = r.q[m];
        // k.q of position tt, summed over its PPT threads (PPT = 8, 16 or 32)
        float d = r.k[m].x * r.q[m].x + r.k[m].y * r.q[m].y + r.k[m].z * r.q[m].z + r.k[m].w * r.q[m].w;
        d = lane_group_sum<(PPT < 16 ? PPT : 16)>(d);
        if constexpr (PPT == 32) d += __shfl_xor(d, 16, kWave);
        if ((f % PPT) == 0) sm.gb[B][tt].z = d;
    }
#pragma unroll
    for (int m = 0; m < StageRegs<LPR>::NV; ++m) {
        const int f = j + 256 * m, tt = f / (RPB / 4), rr = 4 * (f % (RPB / 4));
        *reinterpret_cast<float4*>(&sm.v[B][tt][rr]) = r.v[m];
    }
    if (j < kStageTokens) {
        sm.gb[B][j].x = decay_factor(r.g, p.gate_is_alpha);
        sm.gb[B][j].w = 0.f;
    } else if (j < 2 * kStageTokens) {
        sm.gb[B][j - kStageTokens].y = r.b;
    }
}

template <int LPR, typename T>
__global__ __launch_bounds__(256) void gdr_staged_recurrent_kernel(SeqParams p) {
    constexpr int RPW = 64 / LPR, RPB = kStageWaves * RPW;
    __shared__ __align__(16) StageSmem<LPR> sm;
    const int unit = blockIdx.x;
    const int seq = unit / p.heads, h = unit % p.heads;
    const int j = threadIdx.x, lane = j & 63, w = j >> 6;
    const int li = lane % LPR;
    const int rr = w * RPW + lane / LPR;  // row within the workgroup
    const int i0 = blockIdx.y * RPB;
    const int r = i0 + rr;
    const int dk = p.d_k, dv = p.d_v, H = p.heads;
    const bool row_ok = r < dv;
    int t0, t1;
    seq_bounds(p.cu_seqlens, seq, p.seq_len, t0, t1);
    const int nb = (t1 - t0 + kStageTokens - 1) / kStageTokens;

    float s[16];
    if (p.init && row_ok) {
        load_slice<LPR, true, float>(p.init + ((long)unit * dv + r) * dk, li, dk, s);
    } else {
#pragma unroll
        for (int e = 0; e < 16; ++e) s[e] = 0.f;
    }
    T* op = static_cast<T*>(p.o);

    StageRegs<LPR> regs;
    if (nb > 0) {
        stage_load<LPR, T>(p, h, i0, t0, min(kStageTokens, t1 - t0), j, regs);
        stage_store<LPR>(p, sm, 0, j, regs);
    }
    __syncthreads();
    T* orow = op + (long)h * dv + r;  // o of position t at orow + t * H * dv
    const long ostride = (long)H * dv;
    for (int b = 0; b < nb; ++b) {
        const int B = b & 1;
        const int tb = t0 + b * kStageTokens;
        const int len = min(kStageTokens, t1 - tb);
        const bool more = b + 1 < nb;  // uniform
        if (more) stage_load<LPR, T>(p, h, i0, tb + kStageTokens, min(kStageTokens, t1 - tb - kStageTokens), j, regs);
        for (int tt = 0; tt < len; ++tt) {
            float kr[16], qr[16];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const float4 a = *reinterpret_cast<const float4*>(&sm.k[B][tt][c * 4 * LPR + 4 * li]);
                const float4 e = *reinterpret_cast<const float4*>(&sm.q[B][tt][c * 4 * LPR + 4 * li]);
                kr[4 * c] = a.x, kr[4 * c + 1] = a.y, kr[4 * c + 2] = a.z, kr[4 * c + 3] = a.w;
                qr[4 * c] = e.x, qr[4 * c + 1] = e.y, qr[4 * c + 2] = e.z, qr[4 * c + 3] = e.w;
            }
            const float4 gb = sm.gb[B][tt];  // alpha, beta, k.q
            const float vi = sm.v[B][tt][rr];
            const float sk = lane_group_sum<LPR>(dot16(s, kr));
            const float sq = lane_group_sum<LPR>(dot16(s, qr));
            const float c = gb.y * fmaf(-gb.x, sk, vi);
            const float oi = fmaf(gb.x, sq, c * gb.z);
#pragma unroll
            for (int e = 0; e < 16; ++e) s[e] = fmaf(gb.x, s[e], c * kr[e]);
            if (li == 0 && row_ok) Elem<T>::store(orow, (long)(tb + tt) * ostride, oi);
        }
        if (more) {
            // buffer B ^ 1 was last read in block b - 1, which every wave has
            // left (the barrier below closed it)
            stage_store<LPR>(p, sm, B ^ 1, j, regs);
        }
        __syncthreads();
    }
    if (p.fin && row_ok) store_slice<LPR, true>(p.fin + ((long)unit * dv + r) * dk, li, dk, s);
}

int lanes_per_row(int d_k) { return d_k <= 32 ? 2 : d_k <= 64 ? 4 : d_k <= 128 ? 8 : 16; }

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

template <int LPR, int P, bool VEC, typename T, bool NTL = false>
hipError_t decode_go(const StepParams& sp, int units, int dv, hipStream_t st) {
    constexpr int RPP = 256 / LPR;
    dim3 grid(units, (dv + P * RPP - 1) / (P * RPP));
    hipLaunchKernelGGL((gdr_decode_kernel<LPR, P, VEC, T, NTL>), grid, dim3(256), 0, st, sp);
    return hipGetLastError();
}

// A state of more than kStreamStateBytes is read by non-temporal loads, one
// pass per thread: measured on B = 1024, H = 16, d = 128 (1.07 GB), 5.78-5.81
// TB/s against 5.23-5.29 with two or four passes, 5.15 with plain stores
// and 5.32 with plain loads.  Below it the last-level cache (256 MB) keeps
// much of the state between steps, and plain loads with four passes are
// faster (B = 256, 268 MB: 6.23 against 5.86 TB/s for one pass with
// non-temporal loads and 5.65 with plain ones).
constexpr size_t kStreamStateBytes = size_t(512) << 20;

template <int LPR, bool VEC, typename T>
hipError_t decode_pick_p(const StepParams& sp, int units, int dv, hipStream_t st) {
    constexpr int RPP = 256 / LPR;
    const int passes = (dv + RPP - 1) / RPP;
    const bool stream = VEC && (size_t)units * dv * sp.d_k * sizeof(float) > kStreamStateBytes;
    if (stream) return decode_go<LPR, 1, VEC, T, true>(sp, units, dv, st);
    if (passes >= 4) return decode_go<LPR, 4, VEC, T>(sp, units, dv, st);
    if (passes == 3 || passes == 2) return decode_go<LPR, 2, VEC, T>(sp, units, dv, st);
    return decode_go<LPR, 1, VEC, T>(sp, units, dv, st);
}

template <bool VEC, typename T>
hipError_t decode_pick_lpr(const StepParams& sp, int units, int dk, int dv, hipStream_t st) {
    switch (lanes_per_row(dk)) {
        case 2: return decode_pick_p<2, VEC, T>(sp, units, dv, st);
        case 4: return decode_pick_p<4, VEC, T>(sp, units, dv, st);
        case 8: return decode_pick_p<8, VEC, T>(sp, units, dv, st);
        default: return decode_pick_p<16, VEC, T>(sp, units, dv, st);
    }
}

template <int LPR, int P, bool VEC, typename T>
hipError_t multistep_go(const MultiParams& mp, int units, int dv, hipStream_t st) {
    constexpr int RPP = 256 / LPR;
    dim3 grid(units, (dv + P * RPP - 1) / (P * RPP));
    hipLaunchKernelGGL((gdr_multistep_kernel<LPR, P, VEC, T>), grid, dim3(256), 0, st, mp);
    return hipGetLastError();
}

template <int LPR, bool VEC, typename T>
hipError_t multistep_pick_p(const MultiParams& mp, int units, int dv, hipStream_t st) {
    constexpr int RPP = 256 / LPR;
    // two passes per thread: measured faster than four for the snapshot writes
    const int passes = (dv + RPP - 1) / RPP;
    if (passes >= 2) return multistep_go<LPR, 2, VEC, T>(mp, units, dv, st);
    return multistep_go<LPR, 1, VEC, T>(mp, units, dv, st);
}

template <bool VEC, typename T>
hipError_t multistep_pick_lpr(const MultiParams& mp, int units, int dk, int dv, hipStream_t st) {
    switch (lanes_per_row(dk)) {
        case 2: return multistep_pick_p<2, VEC, T>(mp, units, dv, st);
        case 4: return multistep_pick_p<4, VEC, T>(mp, units, dv, st);
        case 8: return multistep_pick_p<8, VEC, T>(mp, units, dv, st);
        default: return multistep_pick_p<16, VEC, T>(mp, units, dv, st);
    }
}

template <bool VEC, typename T>
hipError_t recurrent_pick_lpr(const SeqParams& sp, int units, int dk, int dv, hipStream_t st) {
    const int lpr = lanes_per_row(dk);
    const int rpw = 64 / lpr;
    dim3 grid(units, (dv + rpw - 1) / rpw);
    switch (lpr) {
        case 2: hipLaunchKernelGGL((gdr_recurrent_kernel<2, VEC, T>), grid, dim3(64), 0, st, sp); break;
        case 4: hipLaunchKernelGGL((gdr_recurrent_kernel<4, VEC, T>), grid, dim3(64), 0, st, sp); break;
        case 8: hipLaunchKernelGGL((gdr_recurrent_kernel<8, VEC, T>), grid, dim3(64), 0, st, sp); break;
        default: hipLaunchKernelGGL((gdr_recurrent_kernel<16, VEC, T>), grid, dim3(64), 0, st, sp); break;
    }
    return hipGetLastError();
}

template <typename T>
hipError_t staged_pick_lpr(const SeqParams& sp, int units, int dk, int dv, hipStream_t st) {
    const int lpr = lanes_per_row(dk);
    const int rpb = kStageWaves * (64 / lpr);
    dim3 grid(units, (dv + rpb - 1) / rpb);
    switch (lpr) {
        case 2: hipLaunchKernelGGL((gdr_staged_recurrent_kernel<2, T>), grid, dim3(256), 0, st, sp); break;
        case 4: hipLaunchKernelGGL((gdr_staged_recurrent_kernel<4, T>), grid, dim3(256), 0, st, sp); break;
        default: hipLaunchKernelGGL((gdr_staged_recurrent_kernel<8, T>), grid, dim3(256), 0, st, sp); break;
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_decode(const rhz_gdr_decode_args& a, hipStream_t st) {
    StepParams sp{a.q, a.k, a.v, a.gate, a.beta, a.state, a.o, a.d_k, a.d_v, a.gate_kind == RHZ_GATE_ALPHA};
    const int units = a.batch * a.heads;
    const size_t ea = a.dtype == RHZ_F32 ? 16 : 8;
    const bool vec = (a.d_k % 4 == 0) && aligned(a.q, ea) && aligned(a.k, ea) && aligned(a.state, 16);
    if (a.dtype == RHZ_F32)
        return vec ? decode_pick_lpr<true, float>(sp, units, a.d_k, a.d_v, st)
                   : decode_pick_lpr<false, float>(sp, units, a.d_k, a.d_v, st);
    return vec ? decode_pick_lpr<true, uint16_t>(sp, units, a.d_k, a.d_v, st)
               : decode_pick_lpr<false, uint16_t>(sp, units, a.d_k, a.d_v, st);
}

hipError_t launch_multistep(const rhz_gdr_multistep_args& a, hipStream_t st) {
    MultiParams mp{a.q, a.k, a.v, a.gate, a.beta, a.state, a.states, a.o,
                   a.steps, a.heads, a.d_k, a.d_v, a.gate_kind == RHZ_GATE_ALPHA};
    const int units = a.batch * a.heads;
    const size_t ea = a.dtype == RHZ_F32 ? 16 : 8;
    const bool vec = (a.d_k % 4 == 0) && aligned(a.q, ea) && aligned(a.k, ea) && aligned(a.state, 16) &&
                     aligned(a.states, 16);
    if (a.dtype == RHZ_F32)
        return vec ? multistep_pick_lpr<true, float>(mp, units, a.d_k, a.d_v, st)
                   : multistep_pick_lpr<false, float>(mp, units, a.d_k, a.d_v, st);
    return vec ? multistep_pick_lpr<true, uint16_t>(mp, units, a.d_k, a.d_v, st)
               : multistep_pick_lpr<false, uint16_t>(mp, units, a.d_k, a.d_v, st);
}

hipError_t launch_recurrent(const rhz_gdr_prefill_args& a, hipStream_t st) {
    SeqParams sp{a.q, a.k, a.v, a.gate, a.beta, a.cu_seqlens, a.initial_state, a.final_state, a.o,
                 a.seq_len, a.heads, a.d_k, a.d_v, a.gate_kind == RHZ_GATE_ALPHA};
    const int units = a.batch * a.heads;
    const size_t ea = a.dtype == RHZ_F32 ? 16 : 8;
    const bool vec = (a.d_k % 4 == 0) && aligned(a.q, ea) && aligned(a.k, ea) &&
                     aligned(a.initial_state, 16) && aligned(a.final_state, 16);
    // positions staged through LDS for d_k <= 128 and whole 4-element pieces
    // of v; the one-position-ahead kernel otherwise
    if (vec && a.d_k <= 128 && a.d_v % 4 == 0 && aligned(a.v, ea))
        return a.dtype == RHZ_F32 ? staged_pick_lpr<float>(sp, units, a.d_k, a.d_v, st)
                                  : staged_pick_lpr<uint16_t>(sp, units, a.d_k, a.d_v, st);
    if (a.dtype == RHZ_F32)
        return vec ? recurrent_pick_lpr<true, float>(sp, units, a.d_k, a.d_v, st)
                   : recurrent_pick_lpr<false, float>(sp, units, a.d_k, a.d_v, st);
    return vec ? recurrent_pick_lpr<true, uint16_t>(sp, units, a.d_k, a.d_v, st)
               : recurrent_pick_lpr<false, uint16_t>(sp, units, a.d_k, a.d_v, st);
}

}  // namespace rhz
