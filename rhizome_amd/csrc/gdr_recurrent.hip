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
// The per-row update and its lane layout are those of gdr_staged.hpp: each
// row of S goes to a group of LPR lanes, and per row and token
//     c_i  = beta * (v_i - alpha * (S_i.k))
//     o_i  = alpha * (S_i.q) + c_i * (k.q)        (= S_i' . q)
//     S_i' = alpha * S_i + c_i * k                (one FMA per element)

#include "gdr_device.hpp"
#include "gdr_internal.hpp"
#include "gdr_staged.hpp"

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
// kStageTokens, for d_k <= 128 (LPR = 2, 4 or 8): one workgroup of four
// waves per (sequence, head, 4 * 64 / LPR rows), running staged_rows
// (gdr_staged.hpp).  The global loads of a block have a whole block's
// compute to arrive.
template <int LPR, typename T, int VPL, int NW>
__global__ __launch_bounds__(NW * 64) void gdr_staged_recurrent_kernel(SeqParams p) {
    __shared__ __align__(16) StageSmem<LPR, VPL, NW> sm;
    const int unit = blockIdx.x;
    const int seq = unit / p.heads, h = unit % p.heads;
    staged_rows<LPR, T, VPL, NW>(p, sm, seq, h, blockIdx.y * StageSmem<LPR, VPL, NW>::RPB, threadIdx.x);
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

// The multistep launch reserves LDS that the kernel does not use, so that at
// most two workgroups (eight waves) share a CU's 160 KiB: the snapshot writes
// then stream from fewer places at once.  B=256 H=16 d=128, 8 positions:
// 459 us at two workgroups per CU against 480 us at the five that the
// registers allow, 483 us at four, 495 us at three and 592 us at one.
constexpr unsigned kMultistepLdsReserve = 64u * 1024u;

template <int LPR, int P, bool VEC, typename T>
hipError_t multistep_go(const MultiParams& mp, int units, int dv, hipStream_t st) {
    constexpr int RPP = 256 / LPR;
    dim3 grid(units, (dv + P * RPP - 1) / (P * RPP));
    hipLaunchKernelGGL((gdr_multistep_kernel<LPR, P, VEC, T>), grid, dim3(256), kMultistepLdsReserve, st, mp);
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
    if (lpr == 8) {
        // d_k in (64, 128]: 16 lanes of 8 columns per row and eight waves of
        // four rows, so that two waves share each SIMD and hide each
        // other's latency along the position chain.
        using Sh = StageShape<16, 8, 8>;
        dim3 grid(units, (dv + Sh::RPB - 1) / Sh::RPB);
        hipLaunchKernelGGL((gdr_staged_recurrent_kernel<16, T, 8, 8>), grid, dim3(Sh::THREADS), 0, st, sp);
        return hipGetLastError();
    }
    const int rpb = kStageWaves * (64 / lpr);
    dim3 grid(units, (dv + rpb - 1) / rpb);
    switch (lpr) {
        case 2: hipLaunchKernelGGL((gdr_staged_recurrent_kernel<2, T, 16, kStageWaves>), grid, dim3(kStageThreads), 0, st, sp); break;
        default: hipLaunchKernelGGL((gdr_staged_recurrent_kernel<4, T, 16, kStageWaves>), grid, dim3(kStageThreads), 0, st, sp); break;
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
