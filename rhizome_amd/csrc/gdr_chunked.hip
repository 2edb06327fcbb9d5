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
// accumulators.  All four state-dependent GEMMs of a chunk (X = [K;Q] S0^T,
// U = T R, O = gamma X_Q + P U, S^T += K^T Uhat) run on 16x16x32 fp16 MFMA
// with the B operand taken straight from the wave's own accumulators: MFMA
// row m of block b stands for index tok(b, m), chosen so that an
// accumulator lane holds 8 consecutive indices of each block pair -- exactly
// the contraction slots of the next product.  So the state-dependent chain
// never leaves the wave; the transposed K operand comes from
// ds_read_b64_tr_b16.
//
// The other six waves prepare the state-independent data one chunk ahead,
// in lockstep with two barriers per chunk:
//   interval A: scan X, R  |  T's off-diagonal 16x16 blocks of chunk c
//               (waves 2, 3)  |  K, Q, V, gates of chunk c+1 into LDS from
//               registers, and chunk c+2 into registers (waves 4-7);
//   interval B: scan U, O, S update  |  K K^T and Q K^T of chunk c+1
//               (waves 2, 3, 6, 7) into A and P, and T's diagonal 16x16
//               blocks by forward substitution in fp32 registers.
// T = (I + A)^-1 is blocked forward substitution: diagonal blocks by
// substitution, then T_ij = -T_ii sum_m A_im T_mj on MFMA.
//
// Operand precision: every GEMM runs on fp16 MFMA (11-bit significands)
// with fp32 accumulation; the carried state is fp32.  K and Q are the bf16
// inputs converted exactly to fp16 (q, k are L2-normalised rows, delta.rs:
// 17-20, so |q.k| <= |q| stays far inside fp16 range); |T| <= 1 for unit
// keys and beta in [0, 1].  S0, R, U and Uhat, whose magnitudes follow the
// data, are rescaled by one power of two per chunk and wave (eS from
// max|S|, eR from max|R|) and the scale is undone exactly in fp32.

#include "gdr_device.hpp"
#include "gdr_internal.hpp"

namespace rhz {
namespace {

constexpr int kTV = 32;           // rows of S per workgroup (two scan waves of 16)
constexpr int kMaxSortSeqs = 4096;
constexpr int kMaxScaleExp = 60;  // bound on the power-of-two operand scales
constexpr int kLDT = 72;          // fp16 row stride of 64-wide LDS tiles

typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

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
    int n_tiles;  // ceil(d_v / 32)
};

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
__device__ __forceinline__ f16x8 pack8(f32x4 lo, f32x4 hi, float s) {
    f16x8 r;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        r[v] = (_Float16)(lo[v] * s);
        r[4 + v] = (_Float16)(hi[v] * s);
    }
    return r;
}

// Eight bf16 values -> eight fp16 values (exact for |x| in the fp16 normal range).
__device__ __forceinline__ uint4 bf16x8_to_f16x8(uint4 u) {
    uint4 r;
    r.x = pack_f16x2(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u));
    r.y = pack_f16x2(__uint_as_float(u.y << 16), __uint_as_float(u.y & 0xffff0000u));
    r.z = pack_f16x2(__uint_as_float(u.z << 16), __uint_as_float(u.z & 0xffff0000u));
    r.w = pack_f16x2(__uint_as_float(u.w << 16), __uint_as_float(u.w & 0xffff0000u));
    return r;
}

// Index (token of a chunk, or key column) carried by MFMA row m of 16-row
// block b: blocks 2c and 2c+1 together cover 32c .. 32c+31, and accumulator
// lane group g (rows 4g..4g+3 of both blocks) holds 32c + 8g + 0..7.
__device__ __forceinline__ int tok(int b, int m) { return 32 * (b >> 1) + 8 * (m >> 2) + 4 * (b & 1) + (m & 3); }

__device__ __forceinline__ void lds_fence() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

__device__ __forceinline__ void seq_bounds(const int* cu, int seq, int seq_len, int& t0, int& t1) {
    if (cu) {
        t0 = min(max(cu[seq], 0), seq_len);
        t1 = min(max(cu[seq + 1], t0), seq_len);
    } else {
        t0 = seq * seq_len;
        t1 = t0 + seq_len;
    }
}

// Chunk-local cumulative log-decay (wave-wide inclusive scan over the 64 tokens).
__device__ __forceinline__ float chunk_cumsum(float g, int lane) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const float y = __shfl_up(g, off, kWave);
        if (lane >= off) g += y;
    }
    return g;
}

// ------------------------------------------------------------ varlen setup
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

// Shared memory of one workgroup.  Buffers indexed [2] are double-buffered
// by chunk parity.  T and P hold zeros above the diagonal blocks for the
// whole kernel.
template <int DK>
struct Smem {
    static constexpr int LDK = DK + 8;  // fp16 row stride of K/Q tiles
    uint16_t k[2][64 * LDK];            // [buf][token][col], fp16
    uint16_t q[2][64 * LDK];
    uint16_t t[2][64 * kLDT];           // T, row-major fp16
    uint16_t p[2][64 * kLDT];           // P, row-major fp16
    uint16_t a[64 * kLDT];              // A, row-major fp16
    uint16_t vt[2][kTV * kLDT];         // V tile transposed [state row][token], bf16
    float gcum[2][64], gam[2][64], gdl[2][64], bs[2][64];
};

// Registers holding one chunk's inputs between its load and its staging
// (loader waves 4-7, lt = thread index within them).
template <int DK>
struct ChunkIn {
    uint4 k[DK / 32], q[DK / 32];  // 16-byte pieces of K and Q rows
    uint4 v;                       // 8 values of the V tile
    float g, b;                    // gate and beta of token lt % 64
};

// Loads are unconditional (indices clamped into the sequence and the row);
// out-of-range values are zeroed when staged.
template <int DK>
__device__ __forceinline__ void load_chunk(const ChunkParams& p, int h, int tb, int te, int i0, int c, int lt,
                                           ChunkIn<DK>& r) {
    constexpr int PPR = DK / 8;
    const int t0 = tb + c * kChunk, last = min(kChunk, te - t0) - 1;
    const int H = p.heads, dk = p.d_k;
#pragma unroll
    for (int u = 0; u < DK / 32; ++u) {
        const int it = lt + 256 * u, row = min(it / PPR, last), c8 = min((it % PPR) * 8, dk - 8);
        const long off = ((long)(t0 + row) * H + h) * dk + c8;
        r.k[u] = *reinterpret_cast<const uint4*>(p.k + off);
        r.q[u] = *reinterpret_cast<const uint4*>(p.q + off);
    }
    {
        const int row = min(lt >> 2, last), c8 = min(i0 + (lt & 3) * 8, p.d_v - 8);
        r.v = *reinterpret_cast<const uint4*>(p.v + ((long)(t0 + row) * H + h) * p.d_v + c8);
    }
    const long gi = (long)(t0 + min(lt & 63, last)) * H + h;
    r.g = p.gate[gi];
    r.b = p.beta[gi];
}

template <int DK>
__device__ __forceinline__ void stage_chunk(const ChunkParams& p, Smem<DK>& sm, int tb, int te, int i0, int c,
                                            int lt, const ChunkIn<DK>& r) {
    constexpr int PPR = DK / 8, LDK = Smem<DK>::LDK;
    const int t0 = tb + c * kChunk, len = min(kChunk, te - t0), b = c & 1;
    const uint4 z = make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int u = 0; u < DK / 32; ++u) {
        const int it = lt + 256 * u, row = it / PPR, c8 = (it % PPR) * 8;
        const bool ok = row < len && c8 < p.d_k;
        *reinterpret_cast<uint4*>(&sm.k[b][row * LDK + c8]) = ok ? bf16x8_to_f16x8(r.k[u]) : z;
        *reinterpret_cast<uint4*>(&sm.q[b][row * LDK + c8]) = ok ? bf16x8_to_f16x8(r.q[u]) : z;
    }
    {
        const int row = lt >> 2, c8 = (lt & 3) * 8;
        const uint4 v = (row < len && i0 + c8 < p.d_v) ? r.v : z;
        const uint32_t wv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            sm.vt[b][(c8 + 2 * e) * kLDT + row] = uint16_t(wv[e]);
            sm.vt[b][(c8 + 2 * e + 1) * kLDT + row] = uint16_t(wv[e] >> 16);
        }
    }
    if (lt < 64) {  // one wave: gates of the 64 tokens
        const float g = lt < len ? log_decay(r.g, p.gate_is_alpha) : 0.f;
        const float G = chunk_cumsum(g, lt);
        const float Glast = __shfl(G, 63, kWave);
        sm.gcum[b][lt] = G;
        sm.gam[b][lt] = __expf(G);
        sm.gdl[b][lt] = __expf(Glast - G);
        sm.bs[b][lt] = lt < len ? r.b : 0.f;
    }
}

// T_ij = -T_ii (sum_{m=j}^{i-1} A_im T_mj) for one 16x16 block of the
// row-major T in tt, by one wave (16x16x16 MFMA).  T_mj enters as the B
// operand through a transposed read.
template <int DK>
__device__ __forceinline__ void t_block(Smem<DK>& sm, uint16_t* tt, int i, int j, int l) {
    const int n = l & 15, kg = l >> 4;
    f32x4 y = {0.f, 0.f, 0.f, 0.f};
    for (int m = j; m < i; ++m) {
        const f16x4 a = ld_f16x4(&sm.a[(16 * i + n) * kLDT + 16 * m + 4 * kg]);
        const s16x4 bt = ld_tr(&tt[(16 * m + 4 * kg + (n >> 2)) * kLDT + 16 * j + 4 * (n & 3)]);
        y = mfma16x16h(a, __builtin_bit_cast(f16x4, bt), y);
    }
    // y[v] = Y[4*kg + v][n]: exactly the B operand of T_ii * Y.
    f16x4 yb;
#pragma unroll
    for (int v = 0; v < 4; ++v) yb[v] = (_Float16)y[v];
    f32x4 t = {0.f, 0.f, 0.f, 0.f};
    t = mfma16x16h(ld_f16x4(&tt[(16 * i + n) * kLDT + 16 * i + 4 * kg]), yb, t);
#pragma unroll
    for (int v = 0; v < 4; ++v) tt[(16 * i + 4 * kg + v) * kLDT + 16 * j + n] = f32_to_f16(-t[v]);
}

// K K^T (isQ false) or Q K^T rows rows_a, rows_b of 16-row blocks for chunk
// buffer b: A (strictly lower) or P (lower incl.) with decay and beta applied.
template <int DK>
__device__ __forceinline__ void kk_rows(Smem<DK>& sm, int b, bool isQ, int ra, int rb, int l) {
    constexpr int LDK = Smem<DK>::LDK, NK = DK / 32;
    const int n = l & 15, g = l >> 4;
    const uint16_t* src = isQ ? sm.q[b] : sm.k[b];
    f16x8 fa[NK], fb[NK];
#pragma unroll
    for (int ks = 0; ks < NK; ++ks) {
        fa[ks] = ld_f16x8(&src[(16 * ra + n) * LDK + 32 * ks + 8 * g]);
        fb[ks] = ld_f16x8(&src[(16 * rb + n) * LDK + 32 * ks + 8 * g]);
    }
    const float4 ga = *reinterpret_cast<const float4*>(&sm.gcum[b][16 * ra + 4 * g]);
    const float4 gb = *reinterpret_cast<const float4*>(&sm.gcum[b][16 * rb + 4 * g]);
    const float4 ba = *reinterpret_cast<const float4*>(&sm.bs[b][16 * ra + 4 * g]);
    const float4 bb = *reinterpret_cast<const float4*>(&sm.bs[b][16 * rb + 4 * g]);
    const float gra[4] = {ga.x, ga.y, ga.z, ga.w}, grb[4] = {gb.x, gb.y, gb.z, gb.w};
    const float bra[4] = {ba.x, ba.y, ba.z, ba.w}, brb[4] = {bb.x, bb.y, bb.z, bb.w};
    uint16_t* dst = isQ ? sm.p[b] : sm.a;
#pragma unroll
    for (int bj = 0; bj < 4; ++bj) {
        if (bj > rb) break;
        const float gs = sm.gcum[b][16 * bj + n];
        const int s = 16 * bj + n;
        f16x8 fk[NK];
#pragma unroll
        for (int ks = 0; ks < NK; ++ks) fk[ks] = ld_f16x8(&sm.k[b][(16 * bj + n) * LDK + 32 * ks + 8 * g]);
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            const int bi = half ? rb : ra;
            if (bj > bi) continue;
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < NK; ++ks) acc = mfma16x32h(half ? fb[ks] : fa[ks], fk[ks], acc);
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int r = 16 * bi + 4 * g + v;
                const float d = __expf(fminf((half ? grb[v] : gra[v]) - gs, 0.f));
                float x = d * acc[v];
                if (!isQ) x *= half ? brb[v] : bra[v];
                const bool keep = isQ ? (s <= r) : (s < r);
                dst[r * kLDT + s] = f32_to_f16(keep ? x : 0.f);
            }
        }
    }
}

// Diagonal block blk of T = (I + A)^-1 by forward substitution: lane col
// (0..15) solves column col in fp32 registers.
template <int DK>
__device__ __forceinline__ void t_diag(Smem<DK>& sm, uint16_t* tt, int blk, int col) {
    float arow[16][16];
#pragma unroll
    for (int r = 1; r < 16; ++r) {
        const uint4 u0 = *reinterpret_cast<const uint4*>(&sm.a[(16 * blk + r) * kLDT + 16 * blk]);
        const uint4 u1 = *reinterpret_cast<const uint4*>(&sm.a[(16 * blk + r) * kLDT + 16 * blk + 8]);
        const uint32_t w[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
#pragma unroll
        for (int s = 0; s < 16; ++s)
            arow[r][s] = float(__builtin_bit_cast(_Float16, uint16_t(w[s >> 1] >> (16 * (s & 1)))));
    }
    float t[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) t[r] = r == col ? 1.f : 0.f;
#pragma unroll
    for (int r = 1; r < 16; ++r) {
        float acc = 0.f;
#pragma unroll
        for (int s = 0; s < r; ++s) acc += arow[r][s] * t[s];
        if (r > col) t[r] = -acc;
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) tt[(16 * blk + r) * kLDT + 16 * blk + col] = f32_to_f16(t[r]);
}

// ------------------------------------------------------------ fused kernel
template <int DK>
__global__ __launch_bounds__(512) void gdr_chunk_kernel(ChunkParams p) {
    constexpr int LDK = Smem<DK>::LDK;
    constexpr int NK = DK / 32;  // 32-wide contraction steps over d_k
    constexpr int NJ = DK / 16;  // 16-row blocks of key columns
    __shared__ __align__(16) Smem<DK> sm;

    const int H = p.heads;
    int unit, tile;
    map_block(blockIdx.x, p.batch * H, p.n_tiles, unit, tile);
    const int seqi = unit / H, h = unit - seqi * H;
    const int seq = p.order ? p.order[seqi] : seqi;
    int tb, te;
    seq_bounds(p.cu_seqlens, seq, p.seq_len, tb, te);
    const int nch = (te - tb + kChunk - 1) / kChunk;
    const int i0 = tile * kTV;
    const int tid = threadIdx.x, l = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int dk = p.d_k, dv = p.d_v;

    // T and P start at zero: their blocks above the diagonal are never written.
    for (int it = tid; it < 2 * 2 * 64 * kLDT / 8; it += 512) {
        uint4* base = reinterpret_cast<uint4*>(it < 2 * 64 * kLDT / 8 ? &sm.t[0][0] : &sm.p[0][0]);
        base[it % (2 * 64 * kLDT / 8)] = make_uint4(0, 0, 0, 0);
    }

    if (w < 2) {
        // ------------------------------------------------------ scan waves
        const int n = l & 15, g = l >> 4;
        const int il = 16 * w + n, i = i0 + il;
        const long srow = (((long)seq * H + h) * dv + i) * dk;
        // S[jb][v] = S[i][tok(jb, 4g + v)]
        f32x4 S[NJ];
#pragma unroll
        for (int jb = 0; jb < NJ; ++jb) S[jb] = (f32x4){0.f, 0.f, 0.f, 0.f};
        if (p.init && i < dv) {
#pragma unroll
            for (int J = 0; J < NK; ++J) {
                const int j = 32 * J + 8 * g;
                if (j < dk) {
                    const float4 a = *reinterpret_cast<const float4*>(p.init + srow + j);
                    const float4 c = *reinterpret_cast<const float4*>(p.init + srow + j + 4);
                    S[2 * J] = (f32x4){a.x, a.y, a.z, a.w};
                    S[2 * J + 1] = (f32x4){c.x, c.y, c.z, c.w};
                }
            }
        }
        auto state_max = [&]() {
            float m = 0.f;
#pragma unroll
            for (int jb = 0; jb < NJ; ++jb)
#pragma unroll
                for (int v = 0; v < 4; ++v) m = fmaxf(m, fabsf(S[jb][v]));
            return wave_max(m);
        };
        float smax = state_max();

        for (int c = -1; c < nch; ++c) {
            const bool act = c >= 0;
            const int b = c & 1;
            const int t0 = tb + c * kChunk, len = min(kChunk, te - t0);
            // ---- interval A: X = [K; Q] S0'^T, R, gamma X_Q.
            f32x4 X[8];
            f16x8 Br[2];
            int eR = 0;
            if (act) {
                const int eS = smax > 0.f ? min(max(ilog2f(smax) - 14, -kMaxScaleExp), kMaxScaleExp) : 0;
                f16x8 Bx[NK];
#pragma unroll
                for (int ks = 0; ks < NK; ++ks) Bx[ks] = pack8(S[2 * ks], S[2 * ks + 1], exp2i(-eS));
#pragma unroll
                for (int bk = 0; bk < 8; ++bk) {
                    const uint16_t* src = bk < 4 ? sm.k[b] : sm.q[b];
                    const int row = tok(bk & 3, n);
                    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int ks = 0; ks < NK; ++ks) acc = mfma16x32h(ld_f16x8(&src[row * LDK + 32 * ks + 8 * g]), Bx[ks], acc);
                    X[bk] = acc;
                }
                const float up = exp2i(eS);
                float rmax = 0.f;
#pragma unroll
                for (int bk = 0; bk < 4; ++bk) {
                    const int s0 = 32 * (bk >> 1) + 8 * g + 4 * (bk & 1);
                    const uint2 vv = *reinterpret_cast<const uint2*>(&sm.vt[b][il * kLDT + s0]);
                    const float4 bs = *reinterpret_cast<const float4*>(&sm.bs[b][s0]);
                    const float4 ga = *reinterpret_cast<const float4*>(&sm.gam[b][s0]);
                    const float vf[4] = {__uint_as_float(vv.x << 16), __uint_as_float(vv.x & 0xffff0000u),
                                         __uint_as_float(vv.y << 16), __uint_as_float(vv.y & 0xffff0000u)};
                    const float bv[4] = {bs.x, bs.y, bs.z, bs.w}, gv[4] = {ga.x, ga.y, ga.z, ga.w};
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const float r = bv[v] * (vf[v] - gv[v] * (X[bk][v] * up));
                        X[bk][v] = r;
                        rmax = fmaxf(rmax, fabsf(r));
                    }
                    const float4 gq = *reinterpret_cast<const float4*>(&sm.gam[b][s0]);
                    X[4 + bk][0] *= gq.x * up;
                    X[4 + bk][1] *= gq.y * up;
                    X[4 + bk][2] *= gq.z * up;
                    X[4 + bk][3] *= gq.w * up;
                }
                rmax = wave_max(rmax);
                eR = rmax > 0.f ? min(max(ilog2f(rmax) - 7, -kMaxScaleExp), kMaxScaleExp) : 0;
                const float sR = exp2i(-eR);
                Br[0] = pack8(X[0], X[1], sR);
                Br[1] = pack8(X[2], X[3], sR);
            }
            __syncthreads();
            // ---- interval B: U' = T R', O = gamma X_Q + 2^eR P U', S update.
            if (act) {
                f32x4 U[4];
#pragma unroll
                for (int rb = 0; rb < 4; ++rb) {
                    const int row = tok(rb, n);
                    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int kk = 0; kk < 2; ++kk) acc = mfma16x32h(ld_f16x8(&sm.t[b][row * kLDT + 32 * kk + 8 * g]), Br[kk], acc);
                    U[rb] = acc;
                }
                f16x8 Bu[2], Bh[2];
#pragma unroll
                for (int kk = 0; kk < 2; ++kk) {
                    Bu[kk] = pack8(U[2 * kk], U[2 * kk + 1], 1.f);
                    const float4 d0 = *reinterpret_cast<const float4*>(&sm.gdl[b][32 * kk + 8 * g]);
                    const float4 d1 = *reinterpret_cast<const float4*>(&sm.gdl[b][32 * kk + 8 * g + 4]);
                    f32x4 h0 = U[2 * kk], h1 = U[2 * kk + 1];
                    h0[0] *= d0.x; h0[1] *= d0.y; h0[2] *= d0.z; h0[3] *= d0.w;
                    h1[0] *= d1.x; h1[1] *= d1.y; h1[2] *= d1.z; h1[3] *= d1.w;
                    Bh[kk] = pack8(h0, h1, 1.f);
                }
                const float down = exp2i(-eR), up = exp2i(eR);
#pragma unroll
                for (int rb = 0; rb < 4; ++rb) {
                    const int row = tok(rb, n);
                    f32x4 acc = X[4 + rb];
#pragma unroll
                    for (int v = 0; v < 4; ++v) acc[v] *= down;
#pragma unroll
                    for (int kk = 0; kk < 2; ++kk) acc = mfma16x32h(ld_f16x8(&sm.p[b][row * kLDT + 32 * kk + 8 * g]), Bu[kk], acc);
                    if (i < dv) {
                        const int r0 = 32 * (rb >> 1) + 8 * g + 4 * (rb & 1);
#pragma unroll
                        for (int v = 0; v < 4; ++v)
                            if (r0 + v < len) p.o[((long)(t0 + r0 + v) * H + h) * dv + i] = f32_to_bf16(acc[v] * up);
                    }
                }
                const float sd = sm.gam[b][63] * down;
#pragma unroll
                for (int jb = 0; jb < NJ; ++jb) {
                    f32x4 acc = S[jb];
#pragma unroll
                    for (int v = 0; v < 4; ++v) acc[v] *= sd;
                    const int col = 32 * (jb >> 1) + 8 * (n & 3) + 4 * (jb & 1);
#pragma unroll
                    for (int kk = 0; kk < 2; ++kk) {
                        const int row = 32 * kk + 8 * g + (n >> 2);
                        const s16x4 lo = ld_tr(&sm.k[b][row * LDK + col]);
                        const s16x4 hi = ld_tr(&sm.k[b][(row + 4) * LDK + col]);
                        const f16x8 ka = __builtin_bit_cast(f16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
                        acc = mfma16x32h(ka, Bh[kk], acc);
                    }
#pragma unroll
                    for (int v = 0; v < 4; ++v) acc[v] *= up;
                    S[jb] = acc;
                }
                smax = state_max();
            }
            __syncthreads();
        }
        if (p.fin && i < dv) {
#pragma unroll
            for (int J = 0; J < NK; ++J) {
                const int j = 32 * J + 8 * g;
                if (j < dk) {
                    *reinterpret_cast<float4*>(p.fin + srow + j) =
                        make_float4(S[2 * J][0], S[2 * J][1], S[2 * J][2], S[2 * J][3]);
                    *reinterpret_cast<float4*>(p.fin + srow + j + 4) =
                        make_float4(S[2 * J + 1][0], S[2 * J + 1][1], S[2 * J + 1][2], S[2 * J + 1][3]);
                }
            }
        }
    } else {
        // ------------------------------------------------------ prep waves
        const bool loader = w >= 4;
        const int lt = tid - 256;
        ChunkIn<DK> in;
        if (loader && nch > 0) load_chunk<DK>(p, h, tb, te, i0, 0, lt, in);
        for (int c = -1; c < nch; ++c) {
            const int nx = c + 1;  // chunk staged and prepared in this iteration
            // ---- interval A: off-diagonal T blocks of chunk c (waves 2, 3);
            //      stage chunk c+1, load chunk c+2 (waves 4-7).
            if (loader) {
                if (nx < nch) {
                    stage_chunk<DK>(p, sm, tb, te, i0, nx, lt, in);
                    load_chunk<DK>(p, h, tb, te, i0, min(nx + 1, nch - 1), lt, in);
                }
            } else if (c >= 0) {
                uint16_t* tt = sm.t[c & 1];
                if (w == 2) {
                    t_block<DK>(sm, tt, 1, 0, l);
                    lds_fence();
                    t_block<DK>(sm, tt, 2, 0, l);
                    lds_fence();
                    t_block<DK>(sm, tt, 3, 0, l);
                } else {
                    t_block<DK>(sm, tt, 3, 2, l);
                    t_block<DK>(sm, tt, 2, 1, l);
                    lds_fence();
                    t_block<DK>(sm, tt, 3, 1, l);
                }
            }
            __syncthreads();
            // ---- interval B: K K^T -> A and Q K^T -> P of chunk c+1 (waves
            //      2, 3, 6, 7), then T's diagonal blocks (waves 2, 3).
            if (nx < nch && (w == 2 || w == 3 || w == 6 || w == 7)) {
                const int nb = nx & 1;
                const bool isQ = w >= 6;
                const int ra = (w & 1) ? 1 : 0, rb = (w & 1) ? 2 : 3;
                kk_rows<DK>(sm, nb, isQ, ra, rb, l);
                if (!isQ) {
                    lds_fence();
                    if (l < 32) t_diag<DK>(sm, sm.t[nb], l < 16 ? ra : rb, l & 15);
                }
            }
            __syncthreads();
        }
    }
}

template <int DK>
hipError_t chunked_go(const ChunkParams& cp, int blocks, hipStream_t st) {
    if (blocks > 0) hipLaunchKernelGGL(gdr_chunk_kernel<DK>, dim3(blocks), dim3(512), 0, st, cp);
    return hipGetLastError();
}

}  // namespace

bool chunked_supported(int d_k, int d_v) {
    return d_k >= 8 && d_k <= 128 && d_k % 8 == 0 && d_v >= 8 && d_v % 8 == 0;
}

size_t chunked_workspace_bytes(const rhz_gdr_prefill_args& a) {
    return a.cu_seqlens ? ((sizeof(int) * (size_t)a.batch + 255) & ~size_t(255)) : 0;
}

hipError_t launch_chunked(const rhz_gdr_prefill_args& a, hipStream_t st) {
    ChunkParams cp;
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
    cp.order = nullptr;
    if (a.cu_seqlens) {
        int* order = static_cast<int*>(a.workspace);
        hipLaunchKernelGGL(gdr_varlen_order_kernel, dim3(1), dim3(1024), 0, st, a.cu_seqlens, a.batch, a.seq_len,
                           order);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        cp.order = order;
    }
    const int blocks = a.batch * a.heads * cp.n_tiles;
    if (a.d_k <= 32) return chunked_go<32>(cp, blocks, st);
    if (a.d_k <= 64) return chunked_go<64>(cp, blocks, st);
    return chunked_go<128>(cp, blocks, st);
}

}  // namespace rhz
