// gdr_chunked.hip -- chunked (WY/UT) gated delta-rule prefill for gfx950:
// bf16 q/k/v, fp32 accumulation, fp32 state, one kernel.
//
// Per 64-token chunk with entering state S0 (d_v x d_k), per-token log-decay
// g, cumulative G_r = sum_{u<=r} g_u, gamma_r = exp(G_r) (all relative to the
// chunk start; every exponent below is <= 0):
//
//   A_rs = beta_r exp(G_r - G_s) k_r.k_s   (s < r),   T = (I + A)^-1
//   P_rs = exp(G_r - G_s) q_r.k_s          (s <= r)
//   R    = diag(beta) (V - diag(gamma) K S0^T)
//   U    = T R                              u_r = beta_r (v_r - alpha_r S_{r-1} k_r)
//   O    = diag(gamma) Q S0^T + P U
//   S'   = gamma_last S0 + sum_r exp(G_last - G_r) u_r k_r^T
//
// which is the recurrence of crates/ops/src/delta.rs:94-127 applied to the
// 64 positions of the chunk (S_r = alpha_r S_{r-1} + u_r k_r^T).
//
// One workgroup of 8 waves per (sequence, head, 32 rows of S).  Rows of S
// are independent, so the d_v split is exact, and each of the two "scan"
// waves owns 16 whole rows of S (every key column) in fp32 MFMA
// accumulators.  All four state-dependent GEMMs of a chunk (X = K S0^T,
// O^T = (Q S0^T)^T + U^T P^T, U = T R, S^T += K^T Uhat) run on 16x16x32 fp16
// MFMA with the state-side operand taken straight from the wave's own
// registers: MFMA row m of block b stands for index tok(b, m), chosen so
// that an accumulator lane holds 8 consecutive indices of each block pair --
// exactly the operand slots of the next product.  So the state-dependent
// chain never leaves the wave; the transposed K operand comes from
// ds_read_b64_tr_b16, and O is produced transposed, so that each lane stores
// 4 consecutive outputs of one token.
//
// The other six waves prepare the state-independent data of the next chunk
// into the other half of double-buffered LDS:
//   waves 4-7 (loaders): K, Q, beta V and the gates of chunk c into LDS from
//               registers, chunk c+2 into the same registers (two register
//               sets alternate), then (loaders 0-2) Q K^T's blocks
//               other than wave 3's;
//   wave 2:     K K^T's diagonal blocks, T's diagonal blocks by forward
//               substitution, T's blocks (1,0), (2,0), (3,0);
//   wave 3:     K K^T below the diagonal, Q K^T's last block row, T's
//               blocks (3,2), (2,1), (3,1).
// T = (I + A)^-1 is blocked forward substitution: diagonal blocks by
// substitution, then T_ij = -T_ii sum_m A_im T_mj on MFMA.  There is no
// workgroup barrier in the chunk loop: each role publishes its progress in
// an LDS counter (incremented by one lane, issued after the step's LDS
// accesses, which the LDS performs first) and waits, by polling, for the
// counters it depends on; a
// buffer is refilled only after both scan waves have counted the chunk that
// last used it.  The chunk loop is unrolled by two, so that the
// double-buffer index is a compile-time constant and every LDS address is a
// per-lane base plus an immediate.
//
// Operand precision: every GEMM runs on fp16 MFMA (11-bit significands)
// with fp32 accumulation; the carried state is fp32.  K and Q are the bf16
// inputs converted to fp16 (exact for |x| >= 2^-14; q, k are L2-normalised
// rows, delta.rs:17-20, so |q.k| <= |q| stays far inside fp16 range);
// |T| <= 1 for unit keys and beta in [0, 1].  The state is held as
// S = Stilde 2^F with one exponent F per scan wave; R, U and O are computed
// in the same scale.  F moves by a power of two only when max|Stilde| or
// max|Rtilde| leaves a window that keeps the fp16 operands (Stilde, Rtilde,
// U) far from overflow and underflow, so in steady state no rescaling
// multiply is executed, and every scale change is exact.

#include <mutex>
#include <utility>

#include "gdr_device.hpp"
#include "gdr_internal.hpp"
#include "gdr_staged.hpp"

namespace rhz {

// Launch parameters of the chunked kernel.  The instances with the fused
// prologue (rhz_gdr_local_prefill) are compiled apart, in
// gdr_chunked_pre.hip, which includes this file: compiled with the plain
// instances in one unit, the plain DK = 128 kernel's register allocation
// changed (256 VGPRs and spills instead of 253 and none).
struct ChunkParams {
    const uint16_t* q;
    const uint16_t* k;
    const uint16_t* v;
    const float* gate;
    const float* beta;
    const int* cu_seqlens;
    const float* init;
    float* fin;
    uint16_t* o;
    const int* order;  // [N] longest-first (packed batches), nullptr for dense
    int batch, seq_len, heads, d_k, d_v, gate_is_alpha;
    int n_tiles;     // ceil(d_v / 32)
    int spin_limit;  // polls after which an LDS wait gives up (and is counted)
    // Fused prologue (the kernel's PRE instances, launched when prologue is
    // set): q and k are the raw projections, gate holds alpha logits and beta
    // holds beta logits.
    int prologue;
    const float* a_log;  // [H]; read only by workgroups with tokens
    float q_scale;
};

// The fused-prologue instances' launch and device counters (compiled in
// gdr_chunked_pre.hip).
hipError_t chunked_go_prologue(const ChunkParams& cp, int dk, int blocks, hipStream_t st);
// which: 0 = LDS waits that gave up, 1 = fp16 range errors, 2 = exact reruns.
hipError_t chunked_prologue_counter(int which, unsigned int* count, bool reset);

namespace {

// Number of LDS waits that gave up since the last reset (per device and
// compilation unit: the host adds the two units' counts).
__device__ unsigned int g_sync_timeouts;
// Number of (workgroup, wave) pairs since the last reset in which an fp16
// entry of A or P (the MFMA operands formed from q and k) was NaN,
// infinite or too large for fp16 (|x| >= 65520) and the workgroup's results
// were not recomputed: only the fused-prologue instances count here (their
// q and k rows are normalised in the kernel); the plain instances rerun
// such a tile exactly instead.  The operands formed from v and the state are
// rescaled by powers of two.
__device__ unsigned int g_range_errors;
// Number of workgroups since the last reset that recomputed their rows with
// the fp32 recurrence (staged_rows) because an input left the domain in
// which the fp16 operands are accurate: an entry of A or P out of fp16's
// range or not finite, a key row with |k|^2 > kKeyNormSqMax, a beta outside
// [0, 1], or a decay alpha outside [0, 1] (log-decay above 0 or NaN).
__device__ unsigned int g_exact_reruns;

constexpr int kTV = 32;           // rows of S per workgroup (two scan waves of 16)
constexpr int kMaxSortSeqs = 4096;
constexpr int kMaxScaleExp = 60;  // bound on one rescaling step
constexpr int kMaxStateExp = 96;  // bound on the state exponent F
constexpr int kLDT = 64;          // fp16 row stride of the 64x64 tiles A, T, P
constexpr int kLDV = 68;          // fp32 row stride of the beta V tile
constexpr int kLDD = 20;          // fp32 row stride of A's diagonal blocks
constexpr int kGateWave = 3;      // loader wave (of 4) that processes the gates
// Largest |k|^2 of the chunked path's domain: unit rows (delta.rs:17-20)
// after bf16 rounding (|k|^2 <= (1 + 2^-9)^2), with margin.  Within it, and
// with beta and alpha in [0, 1], |A_rs| <= |k_r||k_s| stays near 1 and T
// stays well inside fp16's range.
constexpr float kKeyNormSqMax = 1.03125f;

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;


// LDS tile addressing.  Rows are unpadded and the 16-byte chunks of a row
// are permuted by an XOR with a GF(2)-linear function of the row index.  The
// functions were chosen by measuring this kernel's access patterns on gfx950
// (MFMA operand reads of rows tok(b, 0..15) and 16t + 0..15 at a 16-byte
// column, transposed 8-byte reads of K^T and T, and the staging and epilogue
// writes) over candidate permutations: with them the 16-byte operand reads
// run at the LDS's full rate, where padded rows or the identity permutation
// lose a factor of two to bank conflicts.  Reads never straddle a chunk.
__device__ __forceinline__ int rbit(int r, int i) { return (r >> i) & 1; }

template <int DK>
struct KQ;  // K and Q tiles: 64 tokens x DK key columns, fp16
template <>
struct KQ<128> {
    static constexpr int LD = 128;
    static __device__ __forceinline__ int off(int r, int j) {
        const int f = (4 * rbit(r, 0)) ^ (14 * rbit(r, 1)) ^ (3 * rbit(r, 2)) ^ (12 * rbit(r, 3)) ^ (2 * rbit(r, 5));
        return r * LD + (((j >> 3) ^ f) << 3) + (j & 7);
    }
};
template <>
struct KQ<64> {
    static constexpr int LD = 64;
    static __device__ __forceinline__ int off(int r, int j) {
        const int f = 2 * rbit(r, 3) | 4 * (rbit(r, 4) ^ rbit(r, 2));
        return r * LD + (((j >> 3) ^ f) << 3) + (j & 7);
    }
};
template <>
struct KQ<32> {
    static constexpr int LD = 40;  // padded by one chunk
    static __device__ __forceinline__ int off(int r, int j) { return r * LD + (((j >> 3) ^ (2 * rbit(r, 4))) << 3) + (j & 7); }
};
// A, T, P tiles: 64 x 64, fp16
__device__ __forceinline__ int toff(int r, int s) {
    const int f = (3 * rbit(r, 0)) ^ rbit(r, 1) ^ (3 * rbit(r, 2)) ^ (6 * rbit(r, 3)) ^ (3 * rbit(r, 4)) ^ (7 * rbit(r, 5));
    return r * kLDT + (((s >> 3) ^ f) << 3) + (s & 7);
}

__device__ __forceinline__ f16x8 ld_f16x8(const uint16_t* p) {
    return __builtin_bit_cast(f16x8, *reinterpret_cast<const uint4*>(p));
}
__device__ __forceinline__ f16x4 ld_f16x4(const uint16_t* p) {
    return __builtin_bit_cast(f16x4, *reinterpret_cast<const uint2*>(p));
}
// ds_read_b64_tr_b16: within each 16-lane group, lane b receives element b%4
// of the 8-byte vectors addressed by lanes 4a + b/4, a = 0..3.
__device__ __forceinline__ s16x4 ld_tr(const uint16_t* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p));
}
__device__ __forceinline__ f32x4 mfma16x32h(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16x16h(f16x4 a, f16x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f16x8 pack8(f32x4 lo, f32x4 hi) {
    f16x8 r;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        r[v] = (_Float16)lo[v];
        r[4 + v] = (_Float16)hi[v];
    }
    return r;
}
__device__ __forceinline__ f16x8 pack8s(f32x4 lo, f32x4 hi, float s) {
    f16x8 r;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        r[v] = (_Float16)(lo[v] * s);
        r[4 + v] = (_Float16)(hi[v] * s);
    }
    return r;
}
__device__ __forceinline__ uint2 pack_bf16x4(f32x4 a) {
    bf16x4 r;
#pragma unroll
    for (int v = 0; v < 4; ++v) r[v] = (__bf16)a[v];  // round to nearest even
    return __builtin_bit_cast(uint2, r);
}
__device__ __forceinline__ uint2 pack_f16x4(f32x4 a) {
    f16x4 r;
#pragma unroll
    for (int v = 0; v < 4; ++v) r[v] = (_Float16)a[v];
    return __builtin_bit_cast(uint2, r);
}
__device__ __forceinline__ f32x4 ld_f32x4(const float* p) {
    const float4 x = *reinterpret_cast<const float4*>(p);
    return (f32x4){x.x, x.y, x.z, x.w};
}

// Two bf16 (one dword) -> two fp16, round to nearest even (exact for
// |x| >= 2^-14 and below the fp16 maximum).
__device__ __forceinline__ uint32_t bf16x2_to_f16x2(uint32_t u) {
    const f16x2 r = {(_Float16)__uint_as_float(u << 16), (_Float16)__uint_as_float(u & 0xffff0000u)};
    return __builtin_bit_cast(uint32_t, r);
}
__device__ __forceinline__ uint4 bf16x8_to_f16x8(uint4 u) {
    return make_uint4(bf16x2_to_f16x2(u.x), bf16x2_to_f16x2(u.y), bf16x2_to_f16x2(u.z), bf16x2_to_f16x2(u.w));
}
// The same with every value multiplied by f in fp32 before the rounding.
__device__ __forceinline__ uint32_t bf16x2_to_f16x2_scaled(uint32_t u, float f) {
    const f16x2 r = {(_Float16)(__uint_as_float(u << 16) * f), (_Float16)(__uint_as_float(u & 0xffff0000u) * f)};
    return __builtin_bit_cast(uint32_t, r);
}
[[maybe_unused]] __device__ __forceinline__ uint4 bf16x8_to_f16x8_scaled(uint4 u, float f) {
    return make_uint4(bf16x2_to_f16x2_scaled(u.x, f), bf16x2_to_f16x2_scaled(u.y, f),
                      bf16x2_to_f16x2_scaled(u.z, f), bf16x2_to_f16x2_scaled(u.w, f));
}
// The prologue's maps in the hardware's approximate forms (v_exp_f32,
// v_log_f32, v_rcp_f32: about 1 ulp each), for the loader waves:
// sigmoid(x) = 1 / (1 + e^-x); softplus(x) = x past 15, else ln(1 + e^x)
// (for x below about -17, 1 + e^x rounds to 1 and the result is 0, an
// absolute error below 4e-8).
__device__ __forceinline__ float fast_sigmoid(float x) { return __builtin_amdgcn_rcpf(1.f + __expf(-x)); }
__device__ __forceinline__ float fast_softplus(float x) { return x > 15.f ? x : __logf(1.f + __expf(x)); }
// Sum of the squares of eight bf16 (products exact in fp32, bf16 dot2).
[[maybe_unused]] __device__ __forceinline__ float sumsq_bf16x8(uint4 u) {
    float a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, u.x), __builtin_bit_cast(bf16x2, u.x), 0.f,
                                              false);
    a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, u.y), __builtin_bit_cast(bf16x2, u.y), a, false);
    a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, u.z), __builtin_bit_cast(bf16x2, u.z), a, false);
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, u.w), __builtin_bit_cast(bf16x2, u.w), a, false);
}

// Index (token of a chunk, or key column) carried by MFMA row m of 16-row
// block b: blocks 2c and 2c+1 together cover 32c .. 32c+31, and accumulator
// lane group g (rows 4g..4g+3 of both blocks) holds 32c + 8g + 0..7.
__device__ __forceinline__ int tok(int b, int m) { return 32 * (b >> 1) + 8 * (m >> 2) + 4 * (b & 1) + (m & 3); }

// Orders a wave's LDS writes before its own later LDS reads of the same
// data.  The hardware performs one wave's LDS operations in order, so this
// needs no wait, only that the compiler keeps the program order; making
// writes visible to other waves is signal()'s job.
__device__ __forceinline__ void lds_fence() { asm volatile("" ::: "memory"); }

// Inclusive prefix sum over the 64 lanes of a wave: shifts within rows of
// 16 lanes, then row 0's total into row 1 and row 2's into row 3
// (row_bcast:15), then rows 0-1's total into rows 2-3 (row_bcast:31).
__device__ __forceinline__ float wave_incl_scan(float x) {
    x += dpp_mov<0x111>(x);
    x += dpp_mov<0x112>(x);
    x += dpp_mov<0x114>(x);
    x += dpp_mov<0x118>(x);
    x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x142, 0xa, 0xf, false));
    x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x143, 0xc, 0xf, false));
    return x;
}
// The same prefix sum restarted at segment boundaries: lane i sums x_j over
// j <= i with seg_j == seg_i (seg non-decreasing over the lanes).  A lane's
// partial sum covers only its own segment's part of its window, so at each
// shift it takes over the source lane's partial sum only when the two lanes
// are in one segment.  Sums of one segment never see values of another, so
// they are the same numbers whatever came before the segment.
template <int CTRL, int ROWS, bool BOUND>
__device__ __forceinline__ float seg_step(float x, float seg) {
    const float sx = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, ROWS, 0xf, BOUND));
    const float ss = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, seg), CTRL, ROWS, 0xf, BOUND));
    return x + (ss == seg ? sx : 0.f);
}
__device__ __forceinline__ float wave_seg_scan(float x, float seg) {
    x = seg_step<0x111, 0xf, true>(x, seg);
    x = seg_step<0x112, 0xf, true>(x, seg);
    x = seg_step<0x114, 0xf, true>(x, seg);
    x = seg_step<0x118, 0xf, true>(x, seg);
    x = seg_step<0x142, 0xa, false>(x, seg);
    x = seg_step<0x143, 0xc, false>(x, seg);
    return x;
}
__device__ __forceinline__ float lane_val(float x, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), lane));
}

// Power-of-two rescaling step for a quantity whose maximum magnitude is m
// (wave-uniform): 0 while floor(log2 m) lies in [lo, hi) or m is 0, else
// the shift that brings the maximum to [2^target, 2^(target+1)), limited so
// that the state exponent F + shift stays within +-kMaxStateExp.
__device__ __forceinline__ int rescale_shift(float m, int lo, int hi, int target, int F) {
    const int e = ilog2f(m);
    if (!(m > 0.f) || (e >= lo && e < hi)) return 0;
    const int s = min(max(e - target, -kMaxScaleExp), kMaxScaleExp);
    return min(max(F + s, -kMaxStateExp), kMaxStateExp) - F;
}

constexpr float pow2f(int e) { return e >= 0 ? float(1ull << e) : 1.f / float(1ull << -e); }

// rescale_shift of the wave maximum of the lanes' maxima loc (each >= 0,
// never NaN).  The wave maximum m has floor(log2 m) in [LO, HI) exactly when
// no lane reaches 2^HI and some lane reaches 2^LO, and m is 0 when no lane
// is above 0, so the common no-shift case is decided by three ballots; the
// maximum itself is formed only when a shift follows.
template <int LO, int HI, int TARGET>
__device__ __forceinline__ int rescale_shift_lanes(float loc, int F) {
    const bool over = __builtin_amdgcn_ballot_w64(loc >= pow2f(HI)) != 0;
    const bool inside = __builtin_amdgcn_ballot_w64(loc >= pow2f(LO)) != 0;
    const bool zero = __builtin_amdgcn_ballot_w64(loc > 0.f) == 0;
    if (zero || (inside && !over)) return 0;
    return rescale_shift(wave_max(loc), LO, HI, TARGET, F);
}

// ------------------------------------------------------------ varlen setup
#ifndef RHZ_CHUNKED_PROLOGUE_TU  // launched by the plain unit's host code only
// Longest-first order of the packed sequences (ties by index), so the
// longest chunk loops start first.  Identity above kMaxSortSeqs sequences.
__global__ __launch_bounds__(1024) void gdr_varlen_order_kernel(const int* cu, int n, int seq_len, int* order) {
    __shared__ int lens[kMaxSortSeqs];
    if (n > kMaxSortSeqs) {
        for (int i = threadIdx.x; i < n; i += 1024) order[i] = i;
        return;
    }
    for (int i = threadIdx.x; i < n; i += 1024) {
        int t0, t1;
        seq_bounds(cu, i, seq_len, t0, t1);
        lens[i] = t1 - t0;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += 1024) {
        const int li = lens[i];
        int rank = 0;
        for (int j = 0; j < n; ++j) {
            const int lj = lens[j];
            rank += (lj > li) || (lj == li && j < i);
        }
        order[rank] = i;
    }
}
#endif

// Workgroup -> (unit = seq-order index * H + h, tile).  Consecutive
// workgroup ids go round-robin to the 8 XCDs, so the tiles of one unit are
// placed 8 ids apart and share that XCD's L2 (every tile of a unit reads the
// same K, Q and gates).
__device__ __forceinline__ void map_block(int bid, int units, int nt, int& unit, int& tile) {
    const int full = (units / 8) * 8 * nt;
    if (bid < full) {
        const int xcd = bid & 7, slot = bid >> 3;
        tile = slot % nt;
        unit = (slot / nt) * 8 + xcd;
    } else {
        const int rem = bid - full;
        unit = (units / 8) * 8 + rem / nt;
        tile = rem % nt;
    }
}

// ------------------------------------------------------------ wave sync
// The waves of a workgroup synchronise through completion counters in LDS
// instead of workgroup barriers, so that every wave waits only for the data
// it consumes and the preparing waves run up to one chunk ahead of the scan.
// Each counter counts (waves x chunks) finished; a wave that finishes a step
// for chunk x adds 1 after its LDS accesses for that step, and a consumer
// waits until the counter reaches (number of producer waves) * (x + 1).  A
// shared count is exact only because the producers of one counter cannot
// drift apart by a chunk (each waits, before its next chunk, for a step that
// needs all of them); the two scan waves can, so each has its own counter.
// Every wait is for a step of an earlier or the same chunk of another role,
// and each role processes its chunks in order, so the waits form an acyclic
// graph; a wait also gives up after spin_limit polls, so the kernel ends even
// if that property were ever broken.  A wait that gives up adds 1 to
// g_sync_timeouts (one lane, a vector atomic), which the host reads through
// rhz_gdr_sync_timeouts: a nonzero count means the results of that launch
// may be wrong.
struct Sync {
    int staged;  // loader waves (4 per chunk): K, Q, beta V, gates in LDS
    int tdiag;   // wave 2 (1 per chunk): K K^T diagonal blocks and T's diagonal blocks
    int aoff;    // wave 3 (1 per chunk): A below the diagonal
    int tfull;   // waves 2, 3 (2 per chunk): T complete
    int pdone;   // loader waves 0-2 (3 per chunk): P's first three block rows
    int pdone3;  // wave 3 (1 per chunk): P's last block row
    int scanned[2];  // scan wave w (1 per chunk): its last read of the chunk's buffers returned
    int rerun;       // nonzero: an input left the fp16 path's domain (set once, read after the loops)
};

// What the exact rerun needs, written by one thread before the chunk loops
// and read after them, so that no register holds it through the loops.
struct RerunArgs {
    SeqParams sp;
    int seq, h, i0;
};
constexpr int kSpinLimit = 1 << 20;

// Adds 1 to a counter once this wave's earlier LDS accesses are performed.
// A CU's LDS performs the LDS operations of all its waves in one global
// order that keeps each wave's issue order, so the add, issued after the
// step's writes (or its last reads of a buffer), is performed after them; a
// wave that sees the count and then reads sees those writes (or writes
// after those reads).  No wait for completion is needed, only that the
// compiler keeps the program order.
__device__ __forceinline__ void signal(int* cnt) {
    asm volatile("" ::: "memory");
    if ((threadIdx.x & 63) == 0) __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    asm volatile("" ::: "memory");
}
// Waits until every counter c[i] >= t[i] (a target <= 0 holds at once).
// Lane i < N polls counter i against t[i] (the other lanes always pass), so
// a poll is one LDS read and one compare however many counters it checks,
// and a waiting wave takes few issue slots from the wave beside it on its
// SIMD.  Polls follow each other without sleeping (measured faster than
// s_sleep between polls).
typedef __attribute__((address_space(3))) int lds_int;
template <int N>
__device__ __forceinline__ void wait_all(int lim, int* const (&c)[N], const int (&t)[N]) {
    const int lane = __lane_id();
    const lds_int* addr = (const lds_int*)c[0];
    int tgt = -0x7fffffff;
#pragma unroll
    for (int i = 0; i < N; ++i)
        if (lane == i) {
            addr = (const lds_int*)c[i];
            tgt = t[i];
        }
    bool met = false;
    for (int spin = 0; spin < lim; ++spin) {
        const int v = __hip_atomic_load(addr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        if (__builtin_amdgcn_ballot_w64(v < tgt) == 0) {
            met = true;
            break;
        }
    }
    if (!met && lane == 0) atomicAdd(&g_sync_timeouts, 1u);
    asm volatile("" ::: "memory");
}
__device__ __forceinline__ void wait_ge(int lim, int* cnt, int target) { wait_all<1>(lim, {cnt}, {target}); }

// Range watch over fp16 operands: both halves of rng keep the running
// maximum of the magnitude bits (sign cleared) of the fp16 values seen, so
// that a half at or above 0x7c00 means an infinity or a NaN -- a value that
// was not finite, or that rounded to infinity (|x| >= 65520).  Two packed
// 16-bit maxima and two ANDs per four values.
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void range_watch(uint32_t& rng, uint2 h) {
    const u16x2 a = __builtin_bit_cast(u16x2, h.x & 0x7fff7fffu);
    const u16x2 b = __builtin_bit_cast(u16x2, h.y & 0x7fff7fffu);
    rng = __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(u16x2, rng),
                                                                 __builtin_elementwise_max(a, b)));
}
// Whether this lane's watch saw such a value.
__device__ __forceinline__ bool range_bad(uint32_t rng) {
    return (rng & 0xffffu) >= 0x7c00u || (rng >> 16) >= 0x7c00u;
}
// One count in g_range_errors when any lane of the wave saw such a value.
[[maybe_unused]] __device__ __forceinline__ void note_range(uint32_t rng) {
    if (__builtin_amdgcn_ballot_w64(range_bad(rng)) != 0 && (threadIdx.x & 63) == 0) atomicAdd(&g_range_errors, 1u);
}

// Shared memory of one workgroup.  Buffers indexed [2] are double-buffered
// by chunk parity.  T and P hold zeros above the diagonal blocks for the
// whole kernel.
template <int DK>
struct Smem {
    uint16_t k[2][64 * KQ<DK>::LD];  // [buf] token x key column, fp16
    uint16_t q[2][64 * KQ<DK>::LD];
    uint16_t t[2][64 * kLDT];        // T
    uint16_t p[2][64 * kLDT];        // P
    uint16_t a[64 * kLDT];           // A, blocks below the diagonal
    float ad[4 * 16 * kLDD];         // A, diagonal 16x16 blocks, fp32
    float vb[2][kTV * kLDV];         // beta_s v_s[i], [state row i][token s]
    float gcum[2][64];               // G_s
    float gam[2][64];                // exp(G_s)
    float gdl[2][64];                // exp(G_last - G_s)
    float nbg[2][64];                // -beta_s exp(G_s)
    float bs[2][64];                 // beta_s
    float dst[2][64];                // exp(G_s - G_{16 floor(s/16)})
    float den[2][64];                // exp(G_{16 floor(s/16) + 15} - G_s)
    float pf[2][16];                 // [4 bi + bj]: exp(G_{16 bi} - G_{16 bj + 15}), bi > bj
    float seg[2][64];                // segment of token s: resets at or before s
    int resets[2];                   // the chunk has a reset (seg is then valid)
    Sync sync;
    RerunArgs rerun_args;
};

// Marks the workgroup for the exact rerun when any lane of the wave saw an
// input outside the fp16 path's domain; the flag is read once every role
// has left its chunk loop.
template <int DK>
__device__ __forceinline__ void flag_rerun(Smem<DK>& sm, bool bad) {
    if (__builtin_amdgcn_ballot_w64(bad) != 0 && (threadIdx.x & 63) == 0)
        __hip_atomic_store(&sm.sync.rerun, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Per-workgroup constants shared by the roles.
struct Unit {
    int h, seq, tb, te, nch, i0;
    float spa;  // fused prologue: softplus(a_log[h])
};

// ------------------------------------------------------------ loader waves
// Registers holding one chunk's inputs between its load and its staging
// (loader waves 4-7, lt = thread index within them).
template <int DK>
struct ChunkIn {
    uint4 k[DK / 32], q[DK / 32];  // 16-byte pieces of K and Q rows
    uint4 v;                       // 8 values of the V tile (token lt / 4)
    float g, b;                    // gate and beta of token lt % 64
    float bv;                      // beta of token lt / 4
};

// Byte offsets of a loader lane's pieces relative to the first token of a
// chunk (row = token within the chunk, clamped to last).
template <int DK>
struct LoadOffsets {
    uint32_t kq[DK / 32], v, g, bv;
    __device__ __forceinline__ void set(const ChunkParams& p, int i0, int lt, int last) {
        constexpr int PPR = DK / 8;
        const uint32_t H = p.heads, dk = p.d_k, dv = p.d_v;
#pragma unroll
        for (int u = 0; u < DK / 32; ++u) {
            const int it = lt + 256 * u, row = min(it / PPR, last), c8 = min((it % PPR) * 8, p.d_k - 8);
            kq[u] = (uint32_t(row) * H * dk + c8) * 2u;
        }
        const int vrow = min(lt >> 2, last);
        v = (uint32_t(vrow) * H * dv + uint32_t(min(i0 + (lt & 3) * 8, p.d_v - 8) - i0)) * 2u;
        g = uint32_t(min(lt & 63, last)) * H * 4u;
        bv = uint32_t(vrow) * H * 4u;
    }
};

template <int DK>
__device__ __forceinline__ void load_chunk(const ChunkParams& p, const Unit& u, int c, const LoadOffsets<DK>& o,
                                           ChunkIn<DK>& r) {
    const size_t t0 = size_t(u.tb) + size_t(c) * kChunk;
    const size_t H = p.heads;
    const char* kb = reinterpret_cast<const char*>(p.k + (t0 * H + u.h) * p.d_k);
    const char* qb = reinterpret_cast<const char*>(p.q + (t0 * H + u.h) * p.d_k);
    const char* vb = reinterpret_cast<const char*>(p.v + (t0 * H + u.h) * p.d_v + u.i0);
    const char* gb = reinterpret_cast<const char*>(p.gate + t0 * H + u.h);
    const char* bb = reinterpret_cast<const char*>(p.beta + t0 * H + u.h);
#pragma unroll
    for (int i = 0; i < DK / 32; ++i) {
        r.k[i] = *reinterpret_cast<const uint4*>(kb + o.kq[i]);
        r.q[i] = *reinterpret_cast<const uint4*>(qb + o.kq[i]);
    }
    r.v = *reinterpret_cast<const uint4*>(vb + o.v);
    r.g = *reinterpret_cast<const float*>(gb + o.g);
    r.b = *reinterpret_cast<const float*>(bb + o.g);
    r.bv = *reinterpret_cast<const float*>(bb + o.bv);
}

// Loads chunk min(c, nch - 1) (past the end the loads repeat the last chunk
// and are not used).  Only the last chunk can be partial: its offsets,
// clamped to its last token, are selected without a branch, so that the
// compiler's wait for one register set never waits for the loads of the
// other.
template <int DK>
__device__ __forceinline__ void load_chunk_any(const ChunkParams& p, const Unit& u, int c, const LoadOffsets<DK>& full,
                                               const LoadOffsets<DK>& lastc, ChunkIn<DK>& r) {
    c = min(c, u.nch - 1);
    const bool is_last = c == u.nch - 1;  // uniform
    LoadOffsets<DK> o;
#pragma unroll
    for (int i = 0; i < DK / 32; ++i) o.kq[i] = is_last ? lastc.kq[i] : full.kq[i];
    o.v = is_last ? lastc.v : full.v;
    o.g = is_last ? lastc.g : full.g;
    o.bv = is_last ? lastc.bv : full.bv;
    load_chunk<DK>(p, u, c, o, r);
}

// The chunk's decay vectors, lane s = token s.  A reset token (is_reset)
// starts a new segment: seg_s counts the resets at or before s, G_s sums
// the log-decays of s's segment up to s (a reset token's own enters as 0),
// and every factor that spans a reset is exactly zero -- exp(G_r - G_s)
// stands for prod_{s < u <= r} alpha_u only where seg_r == seg_s, and
// exp(G_s) for prod_{u <= s} alpha_u only where seg_s == 0.  Everything from
// a reset on is then computed from the same numbers whatever came before
// it.  Tokens past the chunk's end get g = 0 and beta = 0.
template <int DK, int NB, bool SEG>
__device__ __forceinline__ void stage_gates_as(Smem<DK>& sm, int s, float g, float beta, bool rst) {
    const float sg = SEG ? wave_incl_scan(rst ? 1.f : 0.f) : 0.f;  // small integers: exact
    const float G = SEG ? wave_seg_scan(g, sg) : wave_incl_scan(g);
    const float Glast = lane_val(G, 63);
    const float B0 = lane_val(G, 0), B1 = lane_val(G, 16), B2 = lane_val(G, 32), B3 = lane_val(G, 48);
    const float E0 = lane_val(G, 15), E1 = lane_val(G, 31), E2 = lane_val(G, 47);
    const int blk = s >> 4;
    const float Gs = blk == 0 ? B0 : blk == 1 ? B1 : blk == 2 ? B2 : B3;
    const float Ge = blk == 0 ? E0 : blk == 1 ? E1 : blk == 2 ? E2 : Glast;
    float gam = __expf(G), gdl = __expf(Glast - G), dst = __expf(G - Gs), den = __expf(Ge - G);
    float pf = 0.f;
    const int bi = (s & 15) >> 2, bj = s & 3;
    if (s < 16 && bi > bj) {
        const float gi = bi == 1 ? B1 : bi == 2 ? B2 : B3;
        const float gj = bj == 0 ? E0 : bj == 1 ? E1 : E2;
        pf = __expf(gi - gj);
    }
    if constexpr (SEG) {
        const float Slast = lane_val(sg, 63);
        const float SB0 = lane_val(sg, 0), SB1 = lane_val(sg, 16), SB2 = lane_val(sg, 32), SB3 = lane_val(sg, 48);
        const float SE0 = lane_val(sg, 15), SE1 = lane_val(sg, 31), SE2 = lane_val(sg, 47);
        const float Ss = blk == 0 ? SB0 : blk == 1 ? SB1 : blk == 2 ? SB2 : SB3;
        const float Se = blk == 0 ? SE0 : blk == 1 ? SE1 : blk == 2 ? SE2 : Slast;
        gam = sg == 0.f ? gam : 0.f;
        gdl = sg == Slast ? gdl : 0.f;
        dst = sg == Ss ? dst : 0.f;
        den = sg == Se ? den : 0.f;
        const float si = bi == 1 ? SB1 : bi == 2 ? SB2 : SB3;
        const float sj = bj == 0 ? SE0 : bj == 1 ? SE1 : SE2;
        pf = si == sj ? pf : 0.f;
        sm.seg[NB][s] = sg;
    }
    sm.gcum[NB][s] = G;
    sm.gam[NB][s] = gam;
    sm.gdl[NB][s] = gdl;
    sm.nbg[NB][s] = -beta * gam;
    sm.bs[NB][s] = beta;
    sm.dst[NB][s] = dst;
    sm.den[NB][s] = den;
    if (s < 16) sm.pf[NB][s] = pf;
    if (s == 0) sm.resets[NB] = SEG;
}
// PRE: the gate and beta loaded are logits, mapped as the prologue does
// (g = -softplus(a_h) softplus(alpha_logit), beta = sigmoid(beta_logit)).
// The plain gates' domain (beta and alpha in [0, 1]), tracked across
// chunks: gmax is the running maximum of g + 1/2 and |beta - 1/2|, at most
// 1/2 inside it; nan is set by a NaN gate or beta.
struct GateDomain {
    float gmax = 0.f;
    int nan = 0;
    __device__ __forceinline__ bool bad() const { return nan != 0 || !(gmax <= 0.5f); }
};
template <int DK, int NB, bool PRE>
__device__ __forceinline__ void stage_gates(const ChunkParams& p, Smem<DK>& sm, const Unit& u, int s, int len,
                                            const ChunkIn<DK>& r, GateDomain& dom) {
    const float graw = PRE ? -u.spa * fast_softplus(r.g) : log_decay(r.g, p.gate_is_alpha);
    const bool rst = s < len && is_reset(graw);
    const float g = s < len && !rst ? graw : 0.f;
    const float beta = s < len ? (PRE ? fast_sigmoid(r.b) : r.b) : 0.f;
    if constexpr (!PRE) {
        dom.gmax = fmaxf(dom.gmax, fmaxf(graw + 0.5f, fabsf(beta - 0.5f)));
        dom.nan |= __builtin_isunordered(graw, beta) ? 1 : 0;
    }
    if (__builtin_amdgcn_ballot_w64(rst) == 0)
        stage_gates_as<DK, NB, false>(sm, s, g, beta, rst);
    else
        stage_gates_as<DK, NB, true>(sm, s, g, beta, rst);
}

// Chunk inputs from registers into LDS buffer NB: K and Q as fp16, beta V
// transposed, and (GATES: the gate wave) the gates.  Out-of-range rows and columns are
// written as zeros.
//
// PRE (the fused prologue): every K row is L2-normalised and every Q row
// L2-normalised and multiplied by q_scale as it is staged
// (elementwise.rs:125-128, x / max(||x||, 1e-12) * scale, in fp32 before the
// rounding to fp16, the reciprocal norm by v_rsq_f32), and beta comes from
// its logit.  A row's PPR 16-byte pieces lie on PPR consecutive lanes of one
// wave, so its squared norm is a sum over those lanes.
template <int DK, int NB, bool GATES, bool PRE>
__device__ __forceinline__ void stage_chunk(const ChunkParams& p, Smem<DK>& sm, const Unit& un, int len, int i0,
                                            int lt, const ChunkIn<DK>& r, GateDomain& dom) {
    constexpr int PPR = DK / 8;
    if constexpr (PRE) {
        const uint4 z = make_uint4(0, 0, 0, 0);
#pragma unroll
        for (int u = 0; u < DK / 32; ++u) {
            const int it = lt + 256 * u, row = it / PPR, c8 = (it % PPR) * 8;
            const bool ok = row < len && c8 < p.d_k;
            const uint4 kk = ok ? r.k[u] : z, qq = ok ? r.q[u] : z;
            // 1 / max(||x||, 1e-12) as rsq(max(||x||^2, 1e-24))
            const float fk = __builtin_amdgcn_rsqf(fmaxf(lane_group_sum<PPR>(sumsq_bf16x8(kk)), 1e-24f));
            const float fq = p.q_scale * __builtin_amdgcn_rsqf(fmaxf(lane_group_sum<PPR>(sumsq_bf16x8(qq)), 1e-24f));
            *reinterpret_cast<uint4*>(&sm.k[NB][KQ<DK>::off(row, c8)]) = bf16x8_to_f16x8_scaled(kk, fk);
            *reinterpret_cast<uint4*>(&sm.q[NB][KQ<DK>::off(row, c8)]) = bf16x8_to_f16x8_scaled(qq, fq);
        }
        const int row = lt >> 2, c8 = (lt & 3) * 8;
        const bool ok = row < len && i0 + c8 < p.d_v;
        const float bv = fast_sigmoid(r.bv);
        const uint32_t wv[4] = {r.v.x, r.v.y, r.v.z, r.v.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            sm.vb[NB][(c8 + 2 * e) * kLDV + row] = ok ? bv * __uint_as_float(wv[e] << 16) : 0.f;
            sm.vb[NB][(c8 + 2 * e + 1) * kLDV + row] = ok ? bv * __uint_as_float(wv[e] & 0xffff0000u) : 0.f;
        }
        if constexpr (GATES) stage_gates<DK, NB, true>(p, sm, un, lt & 63, len, r, dom);
        return;
    }
    const bool full = len == kChunk && p.d_k == DK && i0 + kTV <= p.d_v;  // uniform
    if (full) {
#pragma unroll
        for (int u = 0; u < DK / 32; ++u) {
            const int it = lt + 256 * u, row = it / PPR, c8 = (it % PPR) * 8;
            *reinterpret_cast<uint4*>(&sm.k[NB][KQ<DK>::off(row, c8)]) = bf16x8_to_f16x8(r.k[u]);
            *reinterpret_cast<uint4*>(&sm.q[NB][KQ<DK>::off(row, c8)]) = bf16x8_to_f16x8(r.q[u]);
        }
        // beta V^T in 8-byte writes of two tokens: lane l (token 2m + odd)
        // and lane l ^ 4 (the other token of the pair, same 8 state rows)
        // swap four values, then the even lane writes rows c8 + 0..3 and
        // the odd lane rows c8 + 4..7, both at tokens 2m, 2m + 1.
        const int row = lt >> 2, c8 = (lt & 3) * 8;
        const bool odd = row & 1;
        const uint32_t wv[4] = {r.v.x, r.v.y, r.v.z, r.v.w};
        float val[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            val[2 * e] = r.bv * __uint_as_float(wv[e] << 16);
            val[2 * e + 1] = r.bv * __uint_as_float(wv[e] & 0xffff0000u);
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            // lane ^ 4: row_half_mirror, then quad_perm [3, 2, 1, 0]
            const float recv = dpp_mov<0x1B>(dpp_mov<0x141>(odd ? val[k] : val[4 + k]));
            const float2 pair = odd ? make_float2(recv, val[4 + k]) : make_float2(val[k], recv);
            *reinterpret_cast<float2*>(&sm.vb[NB][(c8 + k + (odd ? 4 : 0)) * kLDV + row - (odd ? 1 : 0)]) = pair;
        }
    } else {
        const uint4 z = make_uint4(0, 0, 0, 0);
#pragma unroll
        for (int u = 0; u < DK / 32; ++u) {
            const int it = lt + 256 * u, row = it / PPR, c8 = (it % PPR) * 8;
            const bool ok = row < len && c8 < p.d_k;
            *reinterpret_cast<uint4*>(&sm.k[NB][KQ<DK>::off(row, c8)]) = ok ? bf16x8_to_f16x8(r.k[u]) : z;
            *reinterpret_cast<uint4*>(&sm.q[NB][KQ<DK>::off(row, c8)]) = ok ? bf16x8_to_f16x8(r.q[u]) : z;
        }
        const int row = lt >> 2, c8 = (lt & 3) * 8;
        const bool ok = row < len && i0 + c8 < p.d_v;
        const uint32_t wv[4] = {r.v.x, r.v.y, r.v.z, r.v.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            sm.vb[NB][(c8 + 2 * e) * kLDV + row] = ok ? r.bv * __uint_as_float(wv[e] << 16) : 0.f;
            sm.vb[NB][(c8 + 2 * e + 1) * kLDV + row] = ok ? r.bv * __uint_as_float(wv[e] & 0xffff0000u) : 0.f;
        }
    }
    if constexpr (GATES) stage_gates<DK, NB, false>(p, sm, un, lt & 63, len, r, dom);
}

// ------------------------------------------------------------ K K^T, Q K^T
// Scheduling hints: the next n DS reads, MFMAs, ... go into one group.
#define RHZ_SCHED_GROUP(mask, n) __builtin_amdgcn_sched_group_barrier(mask, n, 0)
constexpr int kSchedMfma = 0x008, kSchedDsRead = 0x100;

// Rows 16 blk + 0..15 of a K or Q tile as the 16-byte operand slices of
// lane (n, g): columns 32 ks + 8 g .. + 7.
template <int DK>
__device__ __forceinline__ void load_rows(const uint16_t* src, int blk, int n, int g, f16x8* dst) {
#pragma unroll
    for (int ks = 0; ks < DK / 32; ++ks) dst[ks] = ld_f16x8(&src[KQ<DK>::off(16 * blk + n, 32 * ks + 8 * g)]);
}

// One 16x16 block (BI, BJ), BJ <= BI, of K K^T (ISQ false) or Q K^T for
// chunk buffer NB, formed transposed, out^T = K_BJ Y_BI^T, so that lane
// (n, g) holds out[16 BI + n][16 BJ + 4 g + 0..3].  The block's product is
// 16x16x32 MFMAs over the key columns (kq_mma); load() reads its epilogue
// factors and store() writes it.  Off-diagonal blocks go to A (beta and
// decay applied) or P (decay applied) in fp16; the decay is the product of
// three factors <= 1, exp(G_r - G_{16 BI}) exp(G_{16 BI} - G_{16 BJ + 15})
// exp(G_{16 BJ + 15} - G_s).  Diagonal blocks are masked to s < r (A, kept
// in fp32 for the substitution) or s <= r (P).  The fp16 values pass
// through rng's range watch.  kmax keeps the running maximum of the
// unmasked products of A's diagonal blocks: it bounds max_r |k_r|^2 from
// below by the diagonal entries and is bounded by it (|k_r.k_s| <= |k_r||k_s|).
// A wave forms its several blocks together: every block's factors are read,
// then the blocks' MFMAs are issued interleaved (independent accumulators),
// then every block is stored.
template <int DK, int NB, bool ISQ, int BI, int BJ>
struct KqBlock {
    static constexpr bool diag = BI == BJ;
    float br, Gr, fr;
    f32x4 es;
    __device__ __forceinline__ void load(Smem<DK>& sm, int l) {
        const int n = l & 15, g = l >> 4;
        const int r = 16 * BI + n, s0 = 16 * BJ + 4 * g;
        br = ISQ ? 1.f : sm.bs[NB][r];
        Gr = sm.gcum[NB][r];
        fr = diag ? 0.f : sm.dst[NB][r] * sm.pf[NB][4 * BI + BJ];
        es = ld_f32x4(diag ? &sm.gcum[NB][s0] : &sm.den[NB][s0]);
    }
    __device__ __forceinline__ void store(Smem<DK>& sm, int l, const f32x4& acc, int resets, uint32_t& rng,
                                          float& kmax) const {
        const int n = l & 15, g = l >> 4;
        const int r = 16 * BI + n, s0 = 16 * BJ + 4 * g;
        f32x4 x;
        if constexpr (!diag) {
            const float f = fr * br;
#pragma unroll
            for (int v = 0; v < 4; ++v) x[v] = acc[v] * f * es[v];
            const uint2 h = pack_f16x4(x);
            range_watch(rng, h);
            *reinterpret_cast<uint2*>(&(ISQ ? sm.p[NB] : sm.a)[toff(r, s0)]) = h;
        } else {
            // plain maxima, so that the compiler orders this read of the
            // accumulators after the MFMAs that write them
            if constexpr (!ISQ) kmax = fmaxf(kmax, fmaxf(fmaxf(acc[0], acc[1]), fmaxf(acc[2], acc[3])));
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int s = s0 + v;
                const bool keep = ISQ ? (s <= r) : (s < r);
                x[v] = keep ? acc[v] * br * __expf(Gr - es[v]) : 0.f;
            }
            if (resets) {  // only pairs in one segment (no reset in (s, r])
                const float sr = sm.seg[NB][r];
                const f32x4 ss = ld_f32x4(&sm.seg[NB][s0]);
#pragma unroll
                for (int v = 0; v < 4; ++v) x[v] = ss[v] == sr ? x[v] : 0.f;
            }
            if constexpr (ISQ) {
                const uint2 h = pack_f16x4(x);
                range_watch(rng, h);
                *reinterpret_cast<uint2*>(&sm.p[NB][toff(r, s0)]) = h;
            } else {
                *reinterpret_cast<float4*>(&sm.ad[(16 * BI + n) * kLDD + 4 * g]) = make_float4(x[0], x[1], x[2], x[3]);
            }
        }
    }
};

// acc[i] = X_i Y_i^T over the key columns for NB blocks at once, the
// MFMAs of the blocks interleaved.
template <int DK, int N>
__device__ __forceinline__ void kq_mma(const f16x8* const (&x)[N], const f16x8* const (&y)[N], f32x4 (&acc)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) acc[i] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < DK / 32; ++ks)
#pragma unroll
        for (int i = 0; i < N; ++i) acc[i] = mfma16x32h(x[i][ks], y[i][ks], acc[i]);
}

// a from lane R of each row of 16 lanes (DPP row_newbcast) times t, and the
// same added to acc: one VALU instruction each.  a is only ever written by LDS
// loads, so the DPP source needs no wait states.
template <int R>
__device__ __forceinline__ float bcast_mul(float a, float t) {
    float r;
    asm("v_mul_f32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf" : "=v"(r) : "v"(a), "v"(t), "i"(R));
    return r;
}
template <int R>
__device__ __forceinline__ float bcast_fma(float a, float t, float acc) {
    asm("v_fmac_f32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf" : "+v"(acc) : "v"(a), "v"(t), "i"(R));
    return acc;
}
// Forward substitution t_R = -sum_{s<R} A[R][s] t_s in column order: once t_S
// is final it is folded into the partial sums of every later row R > S, with
// A[R][S] broadcast from the lane that holds row R.  Each row still sums its
// terms in increasing s, but the rows' sums advance together, so the
// dependent chain is one multiply-add per row instead of one per term.
template <int R>
__device__ __forceinline__ void t_diag_init(float* acc, const float* a, const float* t) {
    acc[R] = bcast_mul<R>(a[0], t[0]);
}
template <int S, int R>
__device__ __forceinline__ void t_diag_fold(float* acc, const float* a, const float* t) {
    acc[R] = bcast_fma<R>(a[S], t[S], acc[R]);
}
template <int S, int... R>
__device__ __forceinline__ void t_diag_col(float* t, float* acc, const float* a, int col,
                                           std::integer_sequence<int, R...>) {
    if (S > col) t[S] = -acc[S];
    (t_diag_fold<S, S + 1 + R>(acc, a, t), ...);
}
template <int... S>
__device__ __forceinline__ void t_diag_solve(float* t, const float* a, int col, std::integer_sequence<int, S...>) {
    float acc[16];
    (t_diag_init<S + 1>(acc, a, t), ...);
    (t_diag_col<S + 1>(t, acc, a, col, std::make_integer_sequence<int, 14 - S>{}), ...);
}

// Diagonal blocks of T = (I + A)^-1 by forward substitution in fp32, one
// wave: lane 16 blk + col holds row col of A's diagonal block blk and solves
// column col of T's.
template <int DK, int NB>
__device__ __forceinline__ void t_diag(Smem<DK>& sm, int l) {
    const int blk = l >> 4, col = l & 15;
    float a[16];
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
        const f32x4 x = ld_f32x4(&sm.ad[(16 * blk + col) * kLDD + 4 * q4]);
#pragma unroll
        for (int e = 0; e < 4; ++e) a[4 * q4 + e] = x[e];
    }
    float t[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) t[r] = r == col ? 1.f : 0.f;
    t_diag_solve(t, a, col, std::make_integer_sequence<int, 15>{});
    // 4-byte writes of two columns: lane col and lane col ^ 1 swap eight
    // values, then the even lane writes rows 0..7 and the odd lane rows
    // 8..15, both at columns col & ~1, (col & ~1) + 1.
    const bool odd = col & 1;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const float recv = dpp_mov<0xB1>(odd ? t[k] : t[8 + k]);  // quad_perm [1, 0, 3, 2]
        *reinterpret_cast<uint32_t*>(&sm.t[NB][toff(16 * blk + k + (odd ? 8 : 0), 16 * blk + (col & ~1))]) =
            pack_f16x2(odd ? recv : t[k], odd ? t[8 + k] : recv);
    }
}

// T_ij = -T_ii (sum_{m=j}^{i-1} A_im T_mj) for one 16x16 block of T (buffer
// NB), by one wave (16x16x16 MFMA).  Y = sum A_im T_mj takes T_mj through a
// transposed read; the second product is formed transposed, (T_ii Y)^T =
// Y^T T_ii^T, so that each lane writes 4 consecutive entries of one row.
template <int DK, int NB, int I, int J>
__device__ __forceinline__ void t_block(Smem<DK>& sm, int l) {
    const int n = l & 15, kg = l >> 4;
    uint16_t* tt = sm.t[NB];
    f16x4 a[I - J];
    s16x4 bt[I - J];
#pragma unroll
    for (int m = J; m < I; ++m) {
        a[m - J] = ld_f16x4(&sm.a[toff(16 * I + n, 16 * m + 4 * kg)]);
        bt[m - J] = ld_tr(&tt[toff(16 * m + 4 * kg + (n >> 2), 16 * J + 4 * (n & 3))]);
    }
    const f16x4 tii = ld_f16x4(&tt[toff(16 * I + n, 16 * I + 4 * kg)]);
    f32x4 y = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = J; m < I; ++m) y = mfma16x16h(a[m - J], __builtin_bit_cast(f16x4, bt[m - J]), y);
    // y[v] = Y[4 kg + v][n]: the A operand Y^T of the transposed product.
    f16x4 ya;
#pragma unroll
    for (int v = 0; v < 4; ++v) ya[v] = (_Float16)y[v];
    f32x4 t = {0.f, 0.f, 0.f, 0.f};
    t = mfma16x16h(ya, tii, t);
    // t[v] = (T_ii Y)[n][4 kg + v]
    *reinterpret_cast<uint2*>(&tt[toff(16 * I + n, 16 * J + 4 * kg)]) = pack_f16x4(-t);
}

template <int DK, int NB, int LW>
__device__ __forceinline__ void qk_blocks(Smem<DK>& sm, int l, uint32_t& rng);
template <int DK, int NB>
__device__ __forceinline__ void qk_blocks_w3(Smem<DK>& sm, int l, uint32_t& rng, const f16x8 (&kr)[4][DK / 32]);

// ------------------------------------------------------------ prep roles
// Wave 2, chunk x (buffer B = x & 1): K K^T's diagonal blocks and T's
// diagonal blocks, then T_10, T_20, T_30.
template <int DK, int B>
__device__ __forceinline__ void prep_wave2(Smem<DK>& sm, int x, int l, int lim, float& kmax) {
    constexpr int NK = DK / 32;
    const int n = l & 15, g = l >> 4;
    // K[B] staged; T[B] was read by the scan and written by both waves for chunk x - 2
    Sync& sy = sm.sync;
    wait_all<4>(lim, {&sy.staged, &sy.scanned[0], &sy.scanned[1], &sy.tfull}, {4 * (x + 1), x - 1, x - 1, 2 * (x - 1)});
    f16x8 kr[4][NK];
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) load_rows<DK>(sm.k[B], blk, n, g, kr[blk]);
    uint32_t unused = 0;  // diagonal blocks of A stay fp32
    {
        KqBlock<DK, B, false, 0, 0> b0;
        KqBlock<DK, B, false, 1, 1> b1;
        KqBlock<DK, B, false, 2, 2> b2;
        KqBlock<DK, B, false, 3, 3> b3;
        b0.load(sm, l), b1.load(sm, l), b2.load(sm, l), b3.load(sm, l);
        const int resets = __builtin_amdgcn_readfirstlane(sm.resets[B]);
        f32x4 acc[4];
        kq_mma<DK, 4>({kr[0], kr[1], kr[2], kr[3]}, {kr[0], kr[1], kr[2], kr[3]}, acc);
        b0.store(sm, l, acc[0], resets, unused, kmax);
        b1.store(sm, l, acc[1], resets, unused, kmax);
        b2.store(sm, l, acc[2], resets, unused, kmax);
        b3.store(sm, l, acc[3], resets, unused, kmax);
    }
    lds_fence();
    t_diag<DK, B>(sm, l);
    signal(&sm.sync.tdiag);
    wait_ge(lim, &sm.sync.aoff, x + 1);
    t_block<DK, B, 1, 0>(sm, l);
    lds_fence();
    t_block<DK, B, 2, 0>(sm, l);
    lds_fence();
    t_block<DK, B, 3, 0>(sm, l);
    signal(&sm.sync.tfull);
}

// Wave 3, chunk x: K K^T below the diagonal into A, then T_32, T_21, T_31.
template <int DK, int B>
__device__ __forceinline__ void prep_wave3(Smem<DK>& sm, int x, int l, int lim, uint32_t& rng) {
    constexpr int NK = DK / 32;
    const int n = l & 15, g = l >> 4;
    // K[B] staged; A (one buffer) was read by T's blocks of chunk x - 1
    wait_all<2>(lim, {&sm.sync.staged, &sm.sync.tfull}, {4 * (x + 1), 2 * x});
    float unused = 0.f;  // off-diagonal blocks: no norm bound
    f16x8 kr[4][NK];
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) load_rows<DK>(sm.k[B], blk, n, g, kr[blk]);
    {
        KqBlock<DK, B, false, 1, 0> b10;
        KqBlock<DK, B, false, 2, 0> b20;
        KqBlock<DK, B, false, 3, 0> b30;
        KqBlock<DK, B, false, 2, 1> b21;
        KqBlock<DK, B, false, 3, 1> b31;
        KqBlock<DK, B, false, 3, 2> b32;
        b10.load(sm, l), b20.load(sm, l), b30.load(sm, l), b21.load(sm, l), b31.load(sm, l), b32.load(sm, l);
        f32x4 acc[6];
        kq_mma<DK, 6>({kr[0], kr[0], kr[0], kr[1], kr[1], kr[2]}, {kr[1], kr[2], kr[3], kr[2], kr[3], kr[3]}, acc);
        b10.store(sm, l, acc[0], 0, rng, unused);
        b20.store(sm, l, acc[1], 0, rng, unused);
        b30.store(sm, l, acc[2], 0, rng, unused);
        b21.store(sm, l, acc[3], 0, rng, unused);
        b31.store(sm, l, acc[4], 0, rng, unused);
        b32.store(sm, l, acc[5], 0, rng, unused);
    }
    signal(&sm.sync.aoff);
    // Q K^T's last block row (the gate loader's share of P would put it on
    // the chunk's critical loop; this wave waits for the diagonal T blocks
    // here anyway), with K from the registers above
    qk_blocks_w3<DK, B>(sm, l, rng, kr);
    signal(&sm.sync.pdone3);
    wait_ge(lim, &sm.sync.tdiag, x + 1);
    t_block<DK, B, 3, 2>(sm, l);
    t_block<DK, B, 2, 1>(sm, l);
    lds_fence();
    t_block<DK, B, 3, 1>(sm, l);
    signal(&sm.sync.tfull);
}

// Q K^T blocks of loader wave LW (0..2) for buffer NB:
//   LW 0: (0,0) (1,0)   LW 1: (1,1) (2,1)   LW 2: (2,0) (2,2)
// (wave 3 forms the last block row, qk_blocks_w3; the gate loader has none).
template <int DK, int NB, int LW>
__device__ __forceinline__ void qk_blocks(Smem<DK>& sm, int l, uint32_t& rng) {
    constexpr int NK = DK / 32;
    const int n = l & 15, g = l >> 4;
    float unused = 0.f;  // Q K^T: no norm bound
    const int resets = __builtin_amdgcn_readfirstlane(sm.resets[NB]);
    if constexpr (LW == 0) {
        f16x8 x0[NK], y0[NK], y1[NK];
        load_rows<DK>(sm.k[NB], 0, n, g, x0);
        load_rows<DK>(sm.q[NB], 0, n, g, y0);
        load_rows<DK>(sm.q[NB], 1, n, g, y1);
        KqBlock<DK, NB, true, 0, 0> b0;
        KqBlock<DK, NB, true, 1, 0> b1;
        b0.load(sm, l), b1.load(sm, l);
        f32x4 acc[2];
        kq_mma<DK, 2>({x0, x0}, {y0, y1}, acc);
        b0.store(sm, l, acc[0], resets, rng, unused);
        b1.store(sm, l, acc[1], resets, rng, unused);
    } else if constexpr (LW == 1) {
        f16x8 x0[NK], y0[NK], y1[NK];
        load_rows<DK>(sm.k[NB], 1, n, g, x0);
        load_rows<DK>(sm.q[NB], 1, n, g, y0);
        load_rows<DK>(sm.q[NB], 2, n, g, y1);
        KqBlock<DK, NB, true, 1, 1> b0;
        KqBlock<DK, NB, true, 2, 1> b1;
        b0.load(sm, l), b1.load(sm, l);
        f32x4 acc[2];
        kq_mma<DK, 2>({x0, x0}, {y0, y1}, acc);
        b0.store(sm, l, acc[0], resets, rng, unused);
        b1.store(sm, l, acc[1], resets, rng, unused);
    } else {
        static_assert(LW == 2, "loader waves 0-2");
        f16x8 x0[NK], x1[NK], y0[NK];
        load_rows<DK>(sm.k[NB], 0, n, g, x0);
        load_rows<DK>(sm.q[NB], 2, n, g, y0);
        load_rows<DK>(sm.k[NB], 2, n, g, x1);
        KqBlock<DK, NB, true, 2, 0> b0;
        KqBlock<DK, NB, true, 2, 2> b1;
        b0.load(sm, l), b1.load(sm, l);
        f32x4 acc[2];
        kq_mma<DK, 2>({x0, x1}, {y0, y0}, acc);
        b0.store(sm, l, acc[0], resets, rng, unused);
        b1.store(sm, l, acc[1], resets, rng, unused);
    }
}

// Wave 3's Q K^T blocks (3,0) .. (3,3), the last block row, for buffer NB,
// K from the registers of its K K^T step, so that only Q's last 16 rows are
// read.
template <int DK, int NB>
__device__ __forceinline__ void qk_blocks_w3(Smem<DK>& sm, int l, uint32_t& rng, const f16x8 (&kr)[4][DK / 32]) {
    constexpr int NK = DK / 32;
    const int n = l & 15, g = l >> 4;
    float unused = 0.f;  // Q K^T: no norm bound
    const int resets = __builtin_amdgcn_readfirstlane(sm.resets[NB]);
    f16x8 y0[NK];
    load_rows<DK>(sm.q[NB], 3, n, g, y0);
    KqBlock<DK, NB, true, 3, 0> b0;
    KqBlock<DK, NB, true, 3, 1> b1;
    KqBlock<DK, NB, true, 3, 2> b2;
    KqBlock<DK, NB, true, 3, 3> b3;
    b0.load(sm, l), b1.load(sm, l), b2.load(sm, l), b3.load(sm, l);
    f32x4 acc[4];
    kq_mma<DK, 4>({kr[0], kr[1], kr[2], kr[3]}, {y0, y0, y0, y0}, acc);
    b0.store(sm, l, acc[0], resets, rng, unused);
    b1.store(sm, l, acc[1], resets, rng, unused);
    b2.store(sm, l, acc[2], resets, rng, unused);
    b3.store(sm, l, acc[3], resets, rng, unused);
}

// Loader wave LW, chunk x (buffer B = x & 1): stage x from registers, load
// x + 2 into the same registers, then Q K^T of x.  Each register set has
// two chunk periods to arrive.
template <int DK, int B, int LW, bool PRE>
__device__ __forceinline__ void prep_loader(const ChunkParams& p, Smem<DK>& sm, const Unit& u, int x, int lt,
                                            const LoadOffsets<DK>& lo, const LoadOffsets<DK>& lastc,
                                            ChunkIn<DK>& in, uint32_t& rng, GateDomain& dom) {
    // buffer B held chunk x - 2: every reader of it is done (nothing to wait for when x < 2)
    Sync& sy = sm.sync;
    wait_all<6>(p.spin_limit, {&sy.scanned[0], &sy.scanned[1], &sy.pdone, &sy.pdone3, &sy.tdiag, &sy.aoff},
                {x - 1, x - 1, 3 * (x - 1), x - 1, x - 1, x - 1});
    const int len = min(kChunk, u.te - (u.tb + x * kChunk));
    stage_chunk<DK, B, LW == kGateWave, PRE>(p, sm, u, len, u.i0, lt, in, dom);
    signal(&sm.sync.staged);
    load_chunk_any<DK>(p, u, x + 2, lo, lastc, in);
    // every loader waits for all four to have staged x, so that none stages
    // x + 1 first (staged counts 4 per chunk)
    wait_ge(p.spin_limit, &sm.sync.staged, 4 * (x + 1));
    if constexpr (LW != kGateWave) {  // the gate loader's Q K^T blocks are wave 3's
        qk_blocks<DK, B, LW>(sm, lt & 63, rng);
        signal(&sm.sync.pdone);
    }
}

template <int DK, int LW, bool PRE>
__device__ __forceinline__ void loader_loop(const ChunkParams& p, Smem<DK>& sm, const Unit& u, int lt) {
    if (u.nch <= 0) return;
    LoadOffsets<DK> lo, lastc;
    lo.set(p, u.i0, lt, kChunk - 1);
    lastc.set(p, u.i0, lt, u.te - (u.tb + (u.nch - 1) * kChunk) - 1);
    ChunkIn<DK> in0, in1;
    load_chunk_any<DK>(p, u, 0, lo, lastc, in0);
    load_chunk_any<DK>(p, u, 1, lo, lastc, in1);
    uint32_t rng = 0;
    GateDomain dom;
    for (int x = 0; x < u.nch; x += 2) {
        prep_loader<DK, 0, LW, PRE>(p, sm, u, x, lt, lo, lastc, in0, rng, dom);
        if (x + 1 >= u.nch) break;
        prep_loader<DK, 1, LW, PRE>(p, sm, u, x + 1, lt, lo, lastc, in1, rng, dom);
    }
    if constexpr (PRE)
        note_range(rng);
    else
        flag_rerun(sm, range_bad(rng) || (LW == kGateWave && dom.bad()));
}

// ------------------------------------------------------------ scan waves
template <int DK>
struct ScanState {
    f32x4 S[DK / 16];  // S[jb][v] = Stilde[i][tok(jb, 4g + v)],  S = Stilde 2^F
    int F;
    float smax;  // this lane's maximum of |Stilde|
};

template <int DK>
__device__ __forceinline__ float state_max(const ScanState<DK>& st) {
    float m = 0.f;
#pragma unroll
    for (int jb = 0; jb < DK / 16; ++jb)
#pragma unroll
        for (int v = 0; v < 4; ++v) m = fmaxf(m, fabsf(st.S[jb][v]));
    return m;
}

// Chunk c of a scan wave (w = 0, 1) on buffer B = c & 1.
template <int DK, int B>
__device__ __forceinline__ void scan_chunk(const ChunkParams& p, Smem<DK>& sm, const Unit& u, int c, int w, int l,
                                           ScanState<DK>& st) {
    constexpr int NK = DK / 32;  // 32-wide contraction steps over d_k
    constexpr int NJ = DK / 16;  // 16-row blocks of key columns
    const int n = l & 15, g = l >> 4;
    const int il = 16 * w + n;
    const int orow = u.i0 + 16 * w + 4 * g;  // first of the 4 output rows of this lane
    const int H = p.heads, dv = p.d_v;
    const int t0 = u.tb + c * kChunk, len = min(kChunk, u.te - t0);
    // ---- X_K = K Stilde^T -> Rtilde;  O^T <- (Q Stilde^T)^T.
    f32x4 OQ[4];
    f16x8 Br[2];
    int er = 0;
    wait_ge(p.spin_limit, &sm.sync.staged, 4 * (c + 1));
    {
        // Operands of this interval, read ahead of their products.
        f16x8 kx[4][NK];
#pragma unroll
        for (int bk = 0; bk < 4; ++bk)
#pragma unroll
            for (int ks = 0; ks < NK; ++ks) kx[bk][ks] = ld_f16x8(&sm.k[B][KQ<DK>::off(tok(bk, n), 32 * ks + 8 * g)]);
        const int es = rescale_shift_lanes<-12, 14, 13>(st.smax, st.F);
        if (es != 0) {
            const float f = exp2i(-es);
#pragma unroll
            for (int jb = 0; jb < NJ; ++jb) st.S[jb] *= f;
            st.F += es;
        }
        f16x8 Bx[NK];
#pragma unroll
        for (int ks = 0; ks < NK; ++ks) Bx[ks] = pack8(st.S[2 * ks], st.S[2 * ks + 1]);
        __builtin_amdgcn_sched_barrier(0);
        // X_K on MFMA while the Q operands are read.
        f16x8 qx[4][NK];
#pragma unroll
        for (int tb2 = 0; tb2 < 4; ++tb2)
#pragma unroll
            for (int ks = 0; ks < NK; ++ks) qx[tb2][ks] = ld_f16x8(&sm.q[B][KQ<DK>::off(16 * tb2 + n, 32 * ks + 8 * g)]);
        f32x4 XK[4];
#pragma unroll
        for (int bk = 0; bk < 4; ++bk) {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < NK; ++ks) acc = mfma16x32h(kx[bk][ks], Bx[ks], acc);
            XK[bk] = acc;
        }
#pragma unroll
        for (int it = 0; it < 4 * NK; ++it) {
            RHZ_SCHED_GROUP(kSchedDsRead, 1);
            RHZ_SCHED_GROUP(kSchedMfma, 1);
        }
        __builtin_amdgcn_sched_barrier(0);
        f32x4 vv[4], nbg[4];
        float gq[4];
#pragma unroll
        for (int bk = 0; bk < 4; ++bk) {
            const int s0 = 32 * (bk >> 1) + 8 * g + 4 * (bk & 1);
            vv[bk] = ld_f32x4(&sm.vb[B][il * kLDV + s0]);
            nbg[bk] = ld_f32x4(&sm.nbg[B][s0]);
            gq[bk] = sm.gam[B][16 * bk + n];
        }
        // (Q Stilde^T)^T on MFMA while Rtilde = beta V 2^-F - beta gamma X_K
        // is formed.
#pragma unroll
        for (int tb2 = 0; tb2 < 4; ++tb2) {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < NK; ++ks) acc = mfma16x32h(Bx[ks], qx[tb2][ks], acc);
            OQ[tb2] = acc;
        }
        float rmax = 0.f;
        if (st.F == 0) {
#pragma unroll
            for (int bk = 0; bk < 4; ++bk)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const float r = fmaf(nbg[bk][v], XK[bk][v], vv[bk][v]);
                    XK[bk][v] = r;
                    rmax = fmaxf(rmax, fabsf(r));
                }
        } else {
            const float sv = exp2i(-st.F);
#pragma unroll
            for (int bk = 0; bk < 4; ++bk)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const float r = fmaf(nbg[bk][v], XK[bk][v], vv[bk][v] * sv);
                    XK[bk][v] = r;
                    rmax = fmaxf(rmax, fabsf(r));
                }
        }
        er = rescale_shift_lanes<-6, 8, 7>(rmax, st.F);
        if (er == 0) {
            Br[0] = pack8(XK[0], XK[1]);
            Br[1] = pack8(XK[2], XK[3]);
        } else {
            const float f = exp2i(-er);
            Br[0] = pack8s(XK[0], XK[1], f);
            Br[1] = pack8s(XK[2], XK[3], f);
        }
        // O^T starts as gamma_t (Q Stilde^T)^T in the scale of U.
        const float fo = exp2i(-er);
#pragma unroll
        for (int tb2 = 0; tb2 < 4; ++tb2) OQ[tb2] *= gq[tb2] * fo;
    }
    // ---- U = T Rhat, O^T += U^T P^T, S update.
    wait_all<3>(p.spin_limit, {&sm.sync.tfull, &sm.sync.pdone, &sm.sync.pdone3}, {2 * (c + 1), 3 * (c + 1), c + 1});
    {
        const int F1 = st.F + er;
        // T rows (both 32-token halves for rows >= 32), P rows, decays.
        f16x8 tr[6], pr[6];
        f32x4 gd[4];
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) tr[rb] = ld_f16x8(&sm.t[B][toff(tok(rb, n), 8 * g)]);
#pragma unroll
        for (int rb = 2; rb < 4; ++rb) tr[rb + 2] = ld_f16x8(&sm.t[B][toff(tok(rb, n), 32 + 8 * g)]);
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            gd[2 * kk] = ld_f32x4(&sm.gdl[B][32 * kk + 8 * g]);
            gd[2 * kk + 1] = ld_f32x4(&sm.gdl[B][32 * kk + 8 * g + 4]);
        }
        const float sd = sm.gam[B][63] * exp2i(-er);
        __builtin_amdgcn_sched_barrier(0);
        f32x4 U[4];
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
            acc = mfma16x32h(tr[rb], Br[0], acc);
            if (rb >= 2) acc = mfma16x32h(tr[rb + 2], Br[1], acc);
            U[rb] = acc;
        }
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) pr[rb] = ld_f16x8(&sm.p[B][toff(16 * rb + n, 8 * g)]);
#pragma unroll
        for (int rb = 2; rb < 4; ++rb) pr[rb + 2] = ld_f16x8(&sm.p[B][toff(16 * rb + n, 32 + 8 * g)]);
        f16x8 Bu[2], Bh[2];
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            Bu[kk] = pack8(U[2 * kk], U[2 * kk + 1]);
            Bh[kk] = pack8(U[2 * kk] * gd[2 * kk], U[2 * kk + 1] * gd[2 * kk + 1]);
        }
        // S update: K^T through transposed reads, 4 column blocks ahead (the
        // earlier the last read of buffer B, the sooner it is refilled:
        // measured 1.8 % faster than 2 ahead, and faster than 3, 5 or 6).
        s16x4 kt[NJ][4];
        auto kt_load = [&](int jb) {
            const int col = 32 * (jb >> 1) + 8 * (n & 3) + 4 * (jb & 1);
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                const int row = 32 * kk + 8 * g + (n >> 2);
                kt[jb][2 * kk] = ld_tr(&sm.k[B][KQ<DK>::off(row, col)]);
                kt[jb][2 * kk + 1] = ld_tr(&sm.k[B][KQ<DK>::off(row + 4, col)]);
            }
        };
        constexpr int kAhead = NJ < 4 ? NJ : 4;
        // The last read of buffer B is issued in S-update step kLastRead
        // (before the loop when negative); the count issued right after it
        // is performed after it, so the chunk is counted there, ahead of the
        // remaining MFMAs, the output stores and the state maximum.
        constexpr int kLastRead = NJ - 1 - kAhead;
#pragma unroll
        for (int jb = 0; jb < kAhead; ++jb) kt_load(jb);
        if constexpr (kLastRead < 0) signal(&sm.sync.scanned[w]);
        // O^T[tb2] lane (n, g): token 16 tb2 + n, state rows orow + 0..3
        f32x4 O[4];
#pragma unroll
        for (int tb2 = 0; tb2 < 4; ++tb2) {
            f32x4 acc = mfma16x32h(Bu[0], pr[tb2], OQ[tb2]);
            if (tb2 >= 2) acc = mfma16x32h(Bu[1], pr[tb2 + 2], acc);
            O[tb2] = acc;
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int jb = 0; jb < NJ; ++jb) {
            if (jb + kAhead < NJ) kt_load(jb + kAhead);
            if (jb == kLastRead) signal(&sm.sync.scanned[w]);
            f32x4 acc = st.S[jb] * sd;
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                const f16x8 ka = __builtin_bit_cast(
                    f16x8, __builtin_shufflevector(kt[jb][2 * kk], kt[jb][2 * kk + 1], 0, 1, 2, 3, 4, 5, 6, 7));
                acc = mfma16x32h(ka, Bh[kk], acc);
            }
            st.S[jb] = acc;
        }
        // Output: 4 consecutive bf16 of one token per lane and block.
        char* const obase = reinterpret_cast<char*>(p.o + (size_t(t0) * H + u.h) * dv);
        const uint32_t ooff = (uint32_t(n) * H * dv + orow) * 2u;
        const uint32_t tstride = 16u * H * dv * 2u;
        if (F1 != 0) {
            const float fout = exp2i(F1);
#pragma unroll
            for (int tb2 = 0; tb2 < 4; ++tb2) O[tb2] *= fout;
        }
#pragma unroll
        for (int tb2 = 0; tb2 < 4; ++tb2)
            if (16 * tb2 + n < len && orow < dv)
                *reinterpret_cast<uint2*>(obase + ooff + tb2 * tstride) = pack_bf16x4(O[tb2]);
        st.F = F1;
        st.smax = state_max(st);
    }
}

// ------------------------------------------------------------ fused kernel
// Shared memory of the chunk loops, reused by the exact rerun.
template <int DK>
union KernelSmem {
    Smem<DK> chunk;
    StageSmem<8> rerun;  // 16 * 8 = 128 key columns, 32 rows: one tile
};
static_assert(StageSmem<8>::RPB == kTV, "the exact rerun covers one tile of rows");

// Workgroup bid -> its (sequence, head, rows) and token range.
template <bool PRE>
__device__ __forceinline__ Unit make_unit(const ChunkParams& p, int bid) {
    const int H = p.heads;
    int unit, tile;
    map_block(bid, p.batch * H, p.n_tiles, unit, tile);
    const int seqi = unit / H;
    Unit u;
    u.h = unit - seqi * H;
    // (clamped: an order buffer that another call overwrote gives wrong
    // results, never an access outside this call's sequences)
    u.seq = p.order ? min(max(p.order[seqi], 0), p.batch - 1) : seqi;
    seq_bounds(p.cu_seqlens, u.seq, p.seq_len, u.tb, u.te);
    u.nch = (u.te - u.tb + kChunk - 1) / kChunk;
    u.i0 = tile * kTV;
    u.spa = PRE && u.nch > 0 ? softplus_f(p.a_log[u.h]) : 0.f;
    return u;
}

// The exact rerun of a tile whose inputs left the fp16 path's domain: the
// whole workgroup, once every role has left its chunk loop, recomputes the
// tile's rows from the initial state with the fp32 recurrence, overwriting
// the outputs and the final state the chunk loops wrote.  Its arguments
// come from LDS (rerun_args), read before the rerun reuses that memory.
template <int DK>
__device__ __forceinline__ void exact_rerun(KernelSmem<DK>& smu) {
    const RerunArgs ra = smu.chunk.rerun_args;
    __syncthreads();  // every wave has read the flag and the arguments: the LDS is free
    staged_rows<8, uint16_t>(ra.sp, smu.rerun, ra.seq, ra.h, ra.i0, threadIdx.x);
}

// PRE: the fused prologue (raw q, k projections and gate / beta logits).
template <int DK, bool PRE>
__global__ __launch_bounds__(512) void gdr_chunk_kernel(ChunkParams p) {
    constexpr int NK = DK / 32;
    __shared__ __align__(16) KernelSmem<DK> smu;
    Smem<DK>& sm = smu.chunk;

    const int H = p.heads;
    const Unit u = make_unit<PRE>(p, blockIdx.x);
    const int tid = threadIdx.x, l = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int dk = p.d_k, dv = p.d_v;

    // T and P start at zero: their blocks above the diagonal are never written.
    for (int it = tid; it < 2 * 2 * 64 * kLDT / 8; it += 512) {
        uint4* base = reinterpret_cast<uint4*>(it < 2 * 64 * kLDT / 8 ? &sm.t[0][0] : &sm.p[0][0]);
        base[it % (2 * 64 * kLDT / 8)] = make_uint4(0, 0, 0, 0);
    }
    if (tid == 0) {
        sm.sync = Sync{0, 0, 0, 0, 0, 0, {0, 0}, 0};
        if constexpr (!PRE)
            sm.rerun_args = RerunArgs{{p.q, p.k, p.v, p.gate, p.beta, p.cu_seqlens, p.init, p.fin, p.o, p.seq_len,
                                       p.heads, p.d_k, p.d_v, p.gate_is_alpha},
                                      u.seq, u.h, u.i0};
    }
    __syncthreads();  // the only workgroup barrier: the chunk loops sync through sm.sync

    // Every role runs chunks 0 .. nch-1, unrolled by two so that buffer c & 1
    // is a compile-time constant.
    if (w < 2) {
        const int n = l & 15, g = l >> 4;
        const int i = u.i0 + 16 * w + n;
        const size_t srow = ((size_t(u.seq) * H + u.h) * dv + i) * dk;
        ScanState<DK> st;
#pragma unroll
        for (int jb = 0; jb < DK / 16; ++jb) st.S[jb] = (f32x4){0.f, 0.f, 0.f, 0.f};
        if (p.init && i < dv) {
#pragma unroll
            for (int J = 0; J < NK; ++J) {
                const int j = 32 * J + 8 * g;
                if (j < dk) {
                    st.S[2 * J] = ld_f32x4(p.init + srow + j);
                    st.S[2 * J + 1] = ld_f32x4(p.init + srow + j + 4);
                }
            }
        }
        st.F = 0;
        st.smax = state_max(st);
        for (int c = 0; c < u.nch; c += 2) {
            scan_chunk<DK, 0>(p, sm, u, c, w, l, st);
            if (c + 1 < u.nch) scan_chunk<DK, 1>(p, sm, u, c + 1, w, l, st);
        }
        if (p.fin && i < dv) {
            const float f = exp2i(st.F);
#pragma unroll
            for (int J = 0; J < NK; ++J) {
                const int j = 32 * J + 8 * g;
                if (j < dk) {
                    const f32x4 a = st.S[2 * J] * f, c = st.S[2 * J + 1] * f;
                    *reinterpret_cast<float4*>(p.fin + srow + j) = make_float4(a[0], a[1], a[2], a[3]);
                    *reinterpret_cast<float4*>(p.fin + srow + j + 4) = make_float4(c[0], c[1], c[2], c[3]);
                }
            }
        }
    } else if (w == 2) {
        float kmax = 0.f;
        for (int x = 0; x < u.nch; x += 2) {
            prep_wave2<DK, 0>(sm, x, l, p.spin_limit, kmax);
            if (x + 1 < u.nch) prep_wave2<DK, 1>(sm, x + 1, l, p.spin_limit, kmax);
        }
        if constexpr (!PRE) flag_rerun(sm, !(kmax <= kKeyNormSqMax));
    } else if (w == 3) {
        uint32_t rng = 0;
        for (int x = 0; x < u.nch; x += 2) {
            prep_wave3<DK, 0>(sm, x, l, p.spin_limit, rng);
            if (x + 1 < u.nch) prep_wave3<DK, 1>(sm, x + 1, l, p.spin_limit, rng);
        }
        if constexpr (PRE)
            note_range(rng);
        else
            flag_rerun(sm, range_bad(rng));
    } else if (w == 4) {
        loader_loop<DK, 0, PRE>(p, sm, u, tid - 256);
    } else if (w == 5) {
        loader_loop<DK, 1, PRE>(p, sm, u, tid - 256);
    } else if (w == 6) {
        loader_loop<DK, 2, PRE>(p, sm, u, tid - 256);
    } else {
        loader_loop<DK, 3, PRE>(p, sm, u, tid - 256);
    }

    if constexpr (!PRE) {
        __syncthreads();  // every role has left its loop and set its flag
        const int rerun = __hip_atomic_load(&sm.sync.rerun, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        if (rerun != 0) {  // uniform over the workgroup
            if (threadIdx.x == 0) atomicAdd(&g_exact_reruns, 1u);
            exact_rerun<DK>(smu);
        }
    }
}

// The value a counter held when read_counter swapped it (one per device and
// compilation unit).
__device__ unsigned int g_counter_read;

// Reads counter `which` (0: g_sync_timeouts, 1: g_range_errors, 2:
// g_exact_reruns) into
// g_counter_read and, when reset is set, zeroes it in the same atomic
// exchange, so that a count added by a kernel still running elsewhere on the
// device lands either in this read or in the next one, never in neither.
__global__ __launch_bounds__(64) void gdr_counter_swap_kernel(int which, int reset) {
    if (threadIdx.x != 0) return;
    unsigned int* c = which == 0 ? &g_sync_timeouts : which == 1 ? &g_range_errors : &g_exact_reruns;
    g_counter_read = reset ? atomicExch(c, 0u) : __hip_atomic_load(c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Waits for all of the current device's work (every stream, blocking or
// not), then swaps the counter on the null stream and copies the value out.
hipError_t read_counter(int which, unsigned int* count, bool reset) {
    hipError_t e = hipDeviceSynchronize();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(gdr_counter_swap_kernel, dim3(1), dim3(64), 0, nullptr, which, reset ? 1 : 0);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    return hipMemcpyFromSymbol(count, HIP_SYMBOL(g_counter_read), sizeof(unsigned int), 0, hipMemcpyDeviceToHost);
}

#ifndef RHZ_CHUNKED_PROLOGUE_TU
template <int DK>
hipError_t chunked_go(const ChunkParams& cp, int blocks, hipStream_t st) {
    if (blocks <= 0) return hipGetLastError();
    if (cp.prologue) return chunked_go_prologue(cp, DK, blocks, st);
    hipLaunchKernelGGL(HIP_KERNEL_NAME(gdr_chunk_kernel<DK, false>), dim3(blocks), dim3(512), 0, st, cp);
    return hipGetLastError();
}
#endif

}  // namespace

#ifdef RHZ_CHUNKED_PROLOGUE_TU
hipError_t chunked_go_prologue(const ChunkParams& cp, int dk, int blocks, hipStream_t st) {
    if (dk == 32)
        hipLaunchKernelGGL(HIP_KERNEL_NAME(gdr_chunk_kernel<32, true>), dim3(blocks), dim3(512), 0, st, cp);
    else if (dk == 64)
        hipLaunchKernelGGL(HIP_KERNEL_NAME(gdr_chunk_kernel<64, true>), dim3(blocks), dim3(512), 0, st, cp);
    else
        hipLaunchKernelGGL(HIP_KERNEL_NAME(gdr_chunk_kernel<128, true>), dim3(blocks), dim3(512), 0, st, cp);
    return hipGetLastError();
}

hipError_t chunked_prologue_counter(int which, unsigned int* count, bool reset) {
    return read_counter(which, count, reset);
}
#else
bool chunked_supported(int d_k, int d_v) {
    return d_k >= 8 && d_k <= 128 && d_k % 8 == 0 && d_v >= 8 && d_v % 8 == 0;
}

size_t chunked_workspace_bytes(const rhz_gdr_prefill_args& a) {
    return a.cu_seqlens ? ((sizeof(int) * (size_t)a.batch + 255) & ~size_t(255)) : 0;
}

// Both counters are the sum of this unit's and the fused-prologue unit's.
hipError_t chunked_sync_timeouts(unsigned int* count, bool reset) {
    unsigned int a = 0, b = 0;
    hipError_t e = read_counter(0, &a, reset);
    if (e == hipSuccess) e = chunked_prologue_counter(0, &b, reset);
    *count = a + b;
    return e;
}

hipError_t chunked_range_errors(unsigned int* count, bool reset) {
    unsigned int a = 0, b = 0;
    hipError_t e = read_counter(1, &a, reset);
    if (e == hipSuccess) e = chunked_prologue_counter(1, &b, reset);
    *count = a + b;
    return e;
}

// Only the plain instances rerun tiles.
hipError_t chunked_exact_reruns(unsigned int* count, bool reset) { return read_counter(2, count, reset); }

namespace {

// The scratch of rhz_gdr_prefill_noalloc: the longest-first order of up to
// kNoAllocMaxSeqs packed sequences (256 KiB).  Each GPU holds its own copy
// until the process ends, and every call on that GPU shares it.  Host code
// never uses this name as an address: the device address of each GPU's copy
// is looked up once (hipGetSymbolAddress, with that device current) and kept
// in g_scratch_dev.
__device__ __align__(256) int scratch[kNoAllocMaxSeqs];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
int* g_scratch_dev[kMaxDevices] = {};  // written under g_scratch_mu

// Device address of the current device's scratch (looked up on the first
// call on that device).
hipError_t noalloc_scratch(int** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_dev[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        g_scratch_dev[dev] = static_cast<int*>(p);
    }
    *out = g_scratch_dev[dev];
    return hipSuccess;
}

// The chunked launch with the packed-batch order in `order_buf` (room for
// a.batch ints; unused for dense batches).
hipError_t launch_chunked_with(const rhz_gdr_prefill_args& a, hipStream_t st, int spin_limit, int* order_buf,
                               const ChunkPrologue* pro = nullptr);

}  // namespace

hipError_t launch_chunked(const rhz_gdr_prefill_args& a, hipStream_t st, int spin_limit, const ChunkPrologue* pro) {
    return launch_chunked_with(a, st, spin_limit, static_cast<int*>(a.workspace), pro);
}

hipError_t launch_chunked_noalloc(const rhz_gdr_prefill_args& a, hipStream_t st) {
    int* order_buf = nullptr;
    if (a.cu_seqlens) {
        if (a.batch > kNoAllocMaxSeqs) return hipErrorInvalidValue;  // the ABI rejects this first
        const hipError_t e = noalloc_scratch(&order_buf);
        if (e != hipSuccess) return e;
    }
    return launch_chunked_with(a, st, 0, order_buf);
}

namespace {
hipError_t launch_chunked_with(const rhz_gdr_prefill_args& a, hipStream_t st, int spin_limit, int* order_buf,
                               const ChunkPrologue* pro) {
    ChunkParams cp;
    cp.prologue = pro != nullptr;
    cp.a_log = pro ? pro->a_log : nullptr;
    cp.q_scale = pro ? pro->q_scale : 1.f;
    cp.q = static_cast<const uint16_t*>(a.q);
    cp.k = static_cast<const uint16_t*>(a.k);
    cp.v = static_cast<const uint16_t*>(a.v);
    cp.gate = a.gate;
    cp.beta = a.beta;
    cp.cu_seqlens = a.cu_seqlens;
    cp.init = a.initial_state;
    cp.fin = a.final_state;
    cp.o = static_cast<uint16_t*>(a.o);
    cp.batch = a.batch;
    cp.seq_len = a.seq_len;
    cp.heads = a.heads;
    cp.d_k = a.d_k;
    cp.d_v = a.d_v;
    cp.gate_is_alpha = a.gate_kind == RHZ_GATE_ALPHA;
    cp.n_tiles = (a.d_v + kTV - 1) / kTV;
    cp.spin_limit = spin_limit > 0 ? spin_limit : kSpinLimit;
    cp.order = nullptr;
    if (a.cu_seqlens) {
        hipLaunchKernelGGL(gdr_varlen_order_kernel, dim3(1), dim3(1024), 0, st, a.cu_seqlens, a.batch, a.seq_len,
                           order_buf);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        cp.order = order_buf;
    }
    const int blocks = a.batch * a.heads * cp.n_tiles;
    if (a.d_k <= 32) return chunked_go<32>(cp, blocks, st);
    if (a.d_k <= 64) return chunked_go<64>(cp, blocks, st);
    return chunked_go<128>(cp, blocks, st);
}
}  // namespace
#endif  // RHZ_CHUNKED_PROLOGUE_TU

}  // namespace rhz
