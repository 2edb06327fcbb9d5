// gdr_staged.hpp -- the token-sequential fp32 recurrence over a block of
// state rows, with the positions staged through LDS.  Used by
// gdr_staged_recurrent_kernel (the fp32-input prefill) and by the chunked
// kernel's exact rerun of a tile whose inputs leave the fp16 path's domain.
//
// Rows of S are independent (row i only reads v_i and its own row), so each
// row goes to a group of LPR lanes; lane li of a group holds columns
// c*4*LPR + 4*li + e (c, e in 0..3), so every 16-byte load of a wave covers
// whole contiguous row segments.  Per row and token the two dot products
// S_i.k and S_i.q and the shared k.q are summed over the group with a fixed
// butterfly, then (crates/ops/src/delta.rs:104-125)
//     c_i  = beta * (v_i - alpha * (S_i.k))
//     o_i  = alpha * (S_i.q) + c_i * (k.q)        (= S_i' . q)
//     S_i' = alpha * S_i + c_i * k                (one FMA per element)
// so the state is read once and written once per position.
#pragma once

#include "gdr_device.hpp"

namespace rhz {

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

// NT: non-temporal stores (streaming output that is not read back, such as
// the multistep snapshots).
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

// Positions per LDS block, and the default shape of the computing waves
// (four: 4 * 64 / LPR state rows, 16 columns per lane).
constexpr int kStageTokens = 32;
constexpr int kStageWaves = 4;
constexpr int kStageThreads = kStageWaves * kWave;

// The dot product of a lane's VPL columns (four partial sums).
template <int VPL>
__device__ __forceinline__ float dot_lane(const float (&a)[VPL], const float (&b)[VPL]) {
    if constexpr (VPL == 8) {
        float s0 = a[0] * b[0], s1 = a[1] * b[1];
#pragma unroll
        for (int e = 2; e < 8; e += 2) {
            s0 = fmaf(a[e], b[e], s0);
            s1 = fmaf(a[e + 1], b[e + 1], s1);
        }
        return s0 + s1;
    }
    float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll
    for (int c = 0; c < VPL / 4; ++c) {
        s0 += a[4 * c + 0] * b[4 * c + 0];
        s1 += a[4 * c + 1] * b[4 * c + 1];
        s2 += a[4 * c + 2] * b[4 * c + 2];
        s3 += a[4 * c + 3] * b[4 * c + 3];
    }
    return (s0 + s1) + (s2 + s3);
}

// The staging layout of NW computing waves whose rows of S each go to LPR
// lanes holding VPL columns: DKP key columns, RPB rows per workgroup.
template <int LPR, int VPL = 16, int NW = kStageWaves>
struct StageShape {
    static constexpr int DKP = VPL * LPR;        // padded key width
    static constexpr int RPW = 64 / LPR;         // rows per wave
    static constexpr int RPB = NW * RPW;         // state rows per workgroup
    static constexpr int THREADS = NW * kWave;
    static constexpr int PPT = DKP / 4;          // float4 pieces of one position's k (or q)
    static constexpr int KQ4 = kStageTokens * PPT;       // float4 pieces of a block's k (or q)
    static constexpr int V4 = kStageTokens * RPB / 4;    // float4 pieces of a block's v
    static constexpr int NKQ = (KQ4 + THREADS - 1) / THREADS;
    static constexpr int NV = (V4 + THREADS - 1) / THREADS;
    static_assert(VPL % 4 == 0 && VPL * LPR >= 4 && PPT <= 32, "supported staging shapes");
};

template <int LPR, int VPL = 16, int NW = kStageWaves>
struct StageSmem {
    using Shape = StageShape<LPR, VPL, NW>;
    static constexpr int DKP = Shape::DKP;
    static constexpr int RPB = Shape::RPB;
    float k[2][kStageTokens][DKP];
    float q[2][kStageTokens][DKP];
    float v[2][kStageTokens][RPB];
    float4 gb[2][kStageTokens];  // (alpha, beta, k.q, 0)
};

// One block's inputs in registers between their global load and their LDS
// write.  Piece m of thread j is float4 number f = j + THREADS m of the
// block's row-major [token][DKP] k (and q) tile; v likewise over
// [token][RPB].
template <int LPR, int VPL = 16, int NW = kStageWaves>
struct StageRegs {
    using Shape = StageShape<LPR, VPL, NW>;
    float4 k[Shape::NKQ], q[Shape::NKQ], v[Shape::NV];
    float g, b;
};

template <int LPR, int VPL, int NW, typename T>
__device__ __forceinline__ void stage_load(const SeqParams& p, int h, int i0, int tb, int len, int j,
                                           StageRegs<LPR, VPL, NW>& r) {
    using S = StageShape<LPR, VPL, NW>;
    const long H = p.heads;
    const T* kp = static_cast<const T*>(p.k);
    const T* qp = static_cast<const T*>(p.q);
    const T* vp = static_cast<const T*>(p.v);
    const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int m = 0; m < S::NKQ; ++m) {
        const int f = j + S::THREADS * m, tt = f / S::PPT, col = 4 * (f % S::PPT);
        const bool ok = f < S::KQ4 && tt < len && col < p.d_k;
        const long off = ((long)(tb + tt) * H + h) * p.d_k + col;
        r.k[m] = ok ? load4(kp + off) : z;
        r.q[m] = ok ? load4(qp + off) : z;
    }
#pragma unroll
    for (int m = 0; m < S::NV; ++m) {
        const int f = j + S::THREADS * m, tt = f / (S::RPB / 4), rr = 4 * (f % (S::RPB / 4));
        const bool ok = f < S::V4 && tt < len && i0 + rr < p.d_v;
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
template <int LPR, int VPL, int NW>
__device__ __forceinline__ void stage_store(const SeqParams& p, StageSmem<LPR, VPL, NW>& sm, int B, int j,
                                            const StageRegs<LPR, VPL, NW>& r) {
    using S = StageShape<LPR, VPL, NW>;
    constexpr int PPT = S::PPT;  // a position's pieces: a group of PPT consecutive threads
#pragma unroll
    for (int m = 0; m < S::NKQ; ++m) {
        const int f = j + S::THREADS * m, tt = f / PPT, col = 4 * (f % PPT);
        if (S::KQ4 % S::THREADS == 0 || f < S::KQ4) {
            *reinterpret_cast<float4*>(&sm.k[B][tt][col]) = r.k[m];
            *reinterpret_cast<float4*>(&sm.q[B][tt][col]) = r.q[m];
        }
        // k.q of position tt, summed over its PPT threads (PPT = 8, 16 or 32)
        float d = r.k[m].x * r.q[m].x + r.k[m].y * r.q[m].y + r.k[m].z * r.q[m].z + r.k[m].w * r.q[m].w;
        d = lane_group_sum<(PPT < 16 ? PPT : 16)>(d);
        if constexpr (PPT == 32) d += __shfl_xor(d, 16, kWave);
        if ((f % PPT) == 0 && f < S::KQ4) sm.gb[B][tt].z = d;
    }
#pragma unroll
    for (int m = 0; m < S::NV; ++m) {
        const int f = j + S::THREADS * m, tt = f / (S::RPB / 4), rr = 4 * (f % (S::RPB / 4));
        if (S::V4 % S::THREADS == 0 || f < S::V4) *reinterpret_cast<float4*>(&sm.v[B][tt][rr]) = r.v[m];
    }
    if (j < kStageTokens) {
        sm.gb[B][j].x = decay_factor(r.g, p.gate_is_alpha);
        sm.gb[B][j].w = 0.f;
    } else if (j < 2 * kStageTokens) {
        sm.gb[B][j - kStageTokens].y = r.b;
    }
}

// Rows i0 .. i0 + RPB - 1 (those below d_v) of sequence `seq`, head h,
// carried through the whole sequence from the initial state (zero without
// one): o written for every position, the final state at the end.  Threads
// j < THREADS compute; a workgroup's further threads only take part in its
// barriers, so every thread of the workgroup must call this.  Every thread
// loads its share of block b + 1 -- k and q rows of the head, the rows' v,
// the gates -- into registers while the waves run block b from LDS, then
// writes it to the other LDS buffer together with k.q of each position
// (summed once per workgroup instead of once per row).  A wave then reads
// each position's k and q from LDS, sums S_i.k and S_i.q over its row's
// lanes by DPP, and updates its rows.  Lane li of a row's group holds
// columns c*4*LPR + 4*li + e (c < VPL/4, e < 4).
template <int LPR, typename T, int VPL = 16, int NW = kStageWaves>
__device__ __forceinline__ void staged_rows(const SeqParams& p, StageSmem<LPR, VPL, NW>& sm, int seq, int h,
                                            int i0, int j) {
    using Sh = StageShape<LPR, VPL, NW>;
    constexpr int RPW = Sh::RPW;
    const bool active = j < Sh::THREADS;  // uniform per wave
    const int lane = j & 63, w = j >> 6;
    const int li = lane % LPR;
    const int rr = w * RPW + lane / LPR;  // row within the block of rows
    const int r = i0 + rr;
    const int dk = p.d_k, dv = p.d_v, H = p.heads;
    const bool row_ok = active && r < dv;
    const long unit = (long)seq * H + h;
    int t0, t1;
    seq_bounds(p.cu_seqlens, seq, p.seq_len, t0, t1);
    const int nb = (t1 - t0 + kStageTokens - 1) / kStageTokens;

    float s[VPL];
#pragma unroll
    for (int c = 0; c < VPL / 4; ++c) {
        const int col = c * 4 * LPR + 4 * li;
        float4 f = make_float4(0.f, 0.f, 0.f, 0.f);
        if (p.init && row_ok && col < dk) f = load4(p.init + (unit * dv + r) * dk + col);
        s[4 * c] = f.x, s[4 * c + 1] = f.y, s[4 * c + 2] = f.z, s[4 * c + 3] = f.w;
    }
    T* op = static_cast<T*>(p.o);

    StageRegs<LPR, VPL, NW> regs;
    if (nb > 0 && active) {
        stage_load<LPR, VPL, NW, T>(p, h, i0, t0, min(kStageTokens, t1 - t0), j, regs);
        stage_store<LPR, VPL, NW>(p, sm, 0, j, regs);
    }
    __syncthreads();
    T* orow = op + (long)h * dv + r;  // o of position t at orow + t * H * dv
    const long ostride = (long)H * dv;
    for (int b = 0; b < nb; ++b) {
        const int B = b & 1;
        const int tb = t0 + b * kStageTokens;
        const int len = min(kStageTokens, t1 - tb);
        const bool more = b + 1 < nb;  // uniform
        if (active) {
            if (more)
                stage_load<LPR, VPL, NW, T>(p, h, i0, tb + kStageTokens, min(kStageTokens, t1 - tb - kStageTokens),
                                            j, regs);
            for (int tt = 0; tt < len; ++tt) {
                float kr[VPL], qr[VPL];
#pragma unroll
                for (int c = 0; c < VPL / 4; ++c) {
                    const float4 a = *reinterpret_cast<const float4*>(&sm.k[B][tt][c * 4 * LPR + 4 * li]);
                    const float4 e = *reinterpret_cast<const float4*>(&sm.q[B][tt][c * 4 * LPR + 4 * li]);
                    kr[4 * c] = a.x, kr[4 * c + 1] = a.y, kr[4 * c + 2] = a.z, kr[4 * c + 3] = a.w;
                    qr[4 * c] = e.x, qr[4 * c + 1] = e.y, qr[4 * c + 2] = e.z, qr[4 * c + 3] = e.w;
                }
                const float4 gb = sm.gb[B][tt];  // alpha, beta, k.q
                const float vi = sm.v[B][tt][rr];
                const float sk = lane_group_sum<LPR>(dot_lane<VPL>(s, kr));
                const float sq = lane_group_sum<LPR>(dot_lane<VPL>(s, qr));
                const float c = gb.y * fmaf(-gb.x, sk, vi);
                float oi = fmaf(gb.x, sq, c * gb.z);
                // o is formed by every lane, ahead of the store's branch, so
                // that k.q is read with the position's other gates rather
                // than inside the branch (an LDS wait per position there)
                asm volatile("" : "+v"(oi));
#pragma unroll
                for (int e = 0; e < VPL; ++e) s[e] = fmaf(gb.x, s[e], c * kr[e]);
                if (li == 0 && row_ok) Elem<T>::store(orow, (long)(tb + tt) * ostride, oi);
            }
            // buffer B ^ 1 was last read in block b - 1, which every wave has
            // left (the barrier below closed it)
            if (more) stage_store<LPR, VPL, NW>(p, sm, B ^ 1, j, regs);
        }
        __syncthreads();
    }
    if (p.fin && row_ok) {
#pragma unroll
        for (int c = 0; c < VPL / 4; ++c) {
            const int col = c * 4 * LPR + 4 * li;
            if (col < dk)
                *reinterpret_cast<float4*>(p.fin + (unit * dv + r) * dk + col) =
                    make_float4(s[4 * c], s[4 * c + 1], s[4 * c + 2], s[4 * c + 3]);
        }
    }
}

}  // namespace rhz
