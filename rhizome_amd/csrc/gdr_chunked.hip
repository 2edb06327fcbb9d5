// gdr_chunked.hip -- chunked (WY/UT) gated delta-rule prefill for gfx950:
// bf16 q/k/v, fp32 accumulation, fp32 state.
//
// Per 64-token chunk with entering state S0 (d_v x d_k), per-token log-decay
// g, cumulative G_r = sum_{u<=r} g_u, gamma_r = exp(G_r) (all relative to the
// chunk start; every exponent below is <= 0):
//
//   A_rs = beta_r exp(G_r - G_s) k_r.k_s   (s < r),   T = (I + A)^-1
//   P_rs = exp(G_r - G_s) q_r.k_s          (s <= r)
//   R    = diag(beta) (V - diag(gamma) K S0^T)          "pseudo-values"
//   U    = T R                              u_r = beta_r (v_r - alpha_r S_{r-1} k_r)
//   O    = diag(gamma) Q S0^T + P U
//   S'   = gamma_last S0 + sum_r exp(G_last - G_r) u_r k_r^T
//
// which is the recurrence of crates/ops/src/delta.rs:94-127 applied to the
// 64 positions of the chunk (S_r = alpha_r S_{r-1} + u_r k_r^T).
//
// Three launches:
//   gdr_varlen_setup_kernel  (packed batches) chunk offsets of each sequence
//                            and a longest-first sequence order;
//   gdr_chunk_prep_kernel    one workgroup per (chunk, head), all chunks in
//                            parallel: K K^T and Q K^T on bf16 MFMA, T by
//                            blocked forward substitution in LDS (fp32,
//                            16x16 diagonal blocks by substitution, the
//                            off-diagonal blocks on fp32 MFMA), T and P
//                            scaled by powers of two into fp16 range and
//                            stored in fp16 in MFMA A-fragment order;
//   gdr_chunk_scan_kernel    one workgroup per (sequence, head, 32 rows of
//                            S); loops over the chunks, state in MFMA
//                            accumulators, next chunk prefetched into
//                            registers.  Rows of S are independent, so the
//                            d_v split is exact.

#include "gdr_device.hpp"
#include "gdr_internal.hpp"

namespace rhz {
namespace {

constexpr int kTV = 32;            // rows of S per scan workgroup
constexpr int kFragBytes = 8192;   // one 64x64 fp16 matrix in fragment order
constexpr int kSlotBytes = 2 * kFragBytes;  // T then P, per (chunk, head)
constexpr int kMaxSortSeqs = 4096;
constexpr int kMaxScaleExp = 60;   // bound on the power-of-two operand scales

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
    const int* chunk_offsets;  // [N+1] for packed batches, nullptr for dense
    const int* order;          // [N] longest-first, nullptr for dense
    uint8_t* tp;               // kSlotBytes per (chunk slot, head): T' then P', fp16
    int2* scales;              // per (chunk slot, head): (eT, eP), T = 2^eT T', P = 2^eP P'
    int batch, seq_len, heads, d_k, d_v, gate_is_alpha;
    int n_chunks_dense;  // ceil(T / 64) for dense batches
    int n_tiles;         // ceil(d_v / 32)
    long n_slots;        // chunk slots in the workspace (bound on every slot index)
};

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 u) { return __builtin_bit_cast(bf16x8, u); }
__device__ __forceinline__ bf16x8 ld_bf16x8(const uint16_t* p) {
    return as_bf16x8(*reinterpret_cast<const uint4*>(p));
}
__device__ __forceinline__ f16x8 ld_f16x8(const uint16_t* p) {
    return __builtin_bit_cast(f16x8, *reinterpret_cast<const uint4*>(p));
}
__device__ __forceinline__ f32x16 mfma32h(f16x8 a, f16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
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
__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ void seq_bounds(const int* cu, int seq, int seq_len, int& t0, int& t1) {
    if (cu) {
        t0 = min(max(cu[seq], 0), seq_len);
        t1 = min(max(cu[seq + 1], t0), seq_len);
    } else {
        t0 = seq * seq_len;
        t1 = t0 + seq_len;
    }
}

// Chunk-local cumulative log-decay (wave-wide inclusive scan over the 64
// tokens).  Prep and scan kernels call this same function on the same
// inputs, so both see bit-identical G.
__device__ __forceinline__ float chunk_cumsum(float g, int lane) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const float y = __shfl_up(g, off, kWave);
        if (lane >= off) g += y;
    }
    return g;
}

// ------------------------------------------------------------ varlen setup
__global__ __launch_bounds__(1024) void gdr_varlen_setup_kernel(const int* cu, int n, int seq_len,
                                                                int* chunk_offsets, int* order) {
    __shared__ int wsum[16];
    __shared__ int carry;
    __shared__ int lens[kMaxSortSeqs];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    if (tid == 0) carry = 0;
    __syncthreads();
    for (int base = 0; base < n; base += 1024) {
        const int i = base + tid;
        int nc = 0;
        if (i < n) {
            int t0, t1;
            seq_bounds(cu, i, seq_len, t0, t1);
            nc = (t1 - t0 + kChunk - 1) / kChunk;
            if (n <= kMaxSortSeqs) lens[i] = t1 - t0;
        }
        int x = nc;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int y = __shfl_up(x, off, kWave);
            if (lane >= off) x += y;
        }
        if (lane == 63) wsum[wv] = x;
        __syncthreads();
        if (wv == 0) {
            int s = lane < 16 ? wsum[lane] : 0;
#pragma unroll
            for (int off = 1; off < 16; off <<= 1) {
                const int y = __shfl_up(s, off, kWave);
                if (lane >= off) s += y;
            }
            if (lane < 16) wsum[lane] = s;
        }
        __syncthreads();
        const int incl = x + (wv > 0 ? wsum[wv - 1] : 0);
        if (i < n) chunk_offsets[i] = carry + incl - nc;
        __syncthreads();
        if (tid == 1023) carry += incl;
        __syncthreads();
    }
    if (tid == 0) chunk_offsets[n] = carry;
    if (n <= kMaxSortSeqs) {
        for (int i = tid; i < n; i += 1024) {
            const int li = lens[i];
            int rank = 0;
            for (int j = 0; j < n; ++j) {
                const int lj = lens[j];
                rank += (lj > li) || (lj == li && j < i);
            }
            order[rank] = i;
        }
    } else {
        for (int i = tid; i < n; i += 1024) order[i] = i;
    }
}

// Chunk slot -> (sequence, chunk within it).  False for slots past the end.
__device__ __forceinline__ bool slot_to_chunk(const ChunkParams& p, int slot, int& seq, int& ci) {
    if (!p.chunk_offsets) {
        seq = slot / p.n_chunks_dense;
        ci = slot - seq * p.n_chunks_dense;
        return seq < p.batch;
    }
    const int* co = p.chunk_offsets;
    if (slot >= co[p.batch]) return false;  // slot < n_slots holds by the grid
    int lo = 0, hi = p.batch - 1;  // largest seq with co[seq] <= slot
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (co[mid] <= slot) lo = mid;
        else hi = mid - 1;
    }
    seq = lo;
    ci = slot - co[lo];
    return true;
}

// 16x16 (fp32) = X[16x16] * Y[16x16] accumulated on v_mfma_f32_16x16x4_f32.
__device__ __forceinline__ f32x4 mm16_f32(const float* X, int ldx, const float* Y, int ldy, f32x4 acc,
                                          int l) {
    const int m = l & 15, kq = l >> 4;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
        const float a = X[m * ldx + 4 * kk + kq];
        const float b = Y[(4 * kk + kq) * ldy + m];
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc, 0, 0, 0);
    }
    return acc;
}

// -------------------------------------------------------------- chunk prep
// Grid (chunk slots, H), 256 threads.
template <int DK>
__global__ __launch_bounds__(256) void gdr_chunk_prep_kernel(ChunkParams p) {
    constexpr int LDK = DK + 8;  // bf16 row stride of K/Q tiles (16-byte pad)
    constexpr int LDA = 65;      // fp32 row stride of A, T and P
    constexpr int LDY = 17;
    __shared__ __align__(16) uint16_t Ks[64 * LDK];
    __shared__ __align__(16) uint16_t Qs[64 * LDK];
    __shared__ float Am[64 * LDA];
    __shared__ float Tm[64 * LDA];
    __shared__ float Pm[64 * LDA];
    __shared__ float Yt[3 * 16 * LDY];
    __shared__ float Gs[64], Bs[64];
    __shared__ float red[2][4];

    const int slot = blockIdx.x, h = blockIdx.y;
    int seq, ci;
    if (!slot_to_chunk(p, slot, seq, ci)) return;
    int tb, te;
    seq_bounds(p.cu_seqlens, seq, p.seq_len, tb, te);
    const int t0 = tb + ci * kChunk;
    const int len = min(kChunk, te - t0);
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63;
    const int H = p.heads;

    // K and Q rows of the chunk (zero past len and past d_k).
    constexpr int PPR = DK / 8;
    for (int it = tid; it < 64 * PPR; it += 256) {
        const int r = it / PPR, c8 = (it % PPR) * 8;
        uint4 kv = make_uint4(0, 0, 0, 0), qv = make_uint4(0, 0, 0, 0);
        if (r < len && c8 < p.d_k) {
            const long off = ((long)(t0 + r) * H + h) * p.d_k + c8;
            kv = *reinterpret_cast<const uint4*>(p.k + off);
            qv = *reinterpret_cast<const uint4*>(p.q + off);
        }
        *reinterpret_cast<uint4*>(&Ks[r * LDK + c8]) = kv;
        *reinterpret_cast<uint4*>(&Qs[r * LDK + c8]) = qv;
    }
    for (int it = tid; it < 64 * LDA; it += 256) {
        Am[it] = 0.f;
        Tm[it] = 0.f;
    }
    if (w == 0) {
        float g = 0.f, b = 0.f;
        if (l < len) {
            const long gi = (long)(t0 + l) * H + h;
            g = log_decay(p.gate[gi], p.gate_is_alpha);
            b = p.beta[gi];
        }
        Gs[l] = chunk_cumsum(g, l);
        Bs[l] = b;
    }
    __syncthreads();

    // K K^T (strictly lower -> A) and Q K^T (lower incl. -> P) in 16x16
    // blocks; blocks above the diagonal are zero.
    for (int task = w; task < 32; task += 4) {
        const bool isQ = task >= 16;
        const int tb16 = task & 15, bi = tb16 >> 2, bj = tb16 & 3;
        const int s = 16 * bj + (l & 15);
        if (bj > bi) {
            if (isQ) {
#pragma unroll
                for (int vv = 0; vv < 4; ++vv) Pm[(16 * bi + 4 * (l >> 4) + vv) * LDA + s] = 0.f;
            }
            continue;
        }
        const uint16_t* src = isQ ? Qs : Ks;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < DK / 32; ++ks) {
            const bf16x8 a = ld_bf16x8(&src[(16 * bi + (l & 15)) * LDK + 32 * ks + 8 * (l >> 4)]);
            const bf16x8 b = ld_bf16x8(&Ks[(16 * bj + (l & 15)) * LDK + 32 * ks + 8 * (l >> 4)]);
            acc = mfma16(a, b, acc);
        }
#pragma unroll
        for (int vv = 0; vv < 4; ++vv) {
            const int r = 16 * bi + 4 * (l >> 4) + vv;
            if (!isQ) Am[r * LDA + s] = (s < r) ? Bs[r] * __expf(Gs[r] - Gs[s]) * acc[vv] : 0.f;
            else Pm[r * LDA + s] = (s <= r) ? __expf(Gs[r] - Gs[s]) * acc[vv] : 0.f;
        }
    }
    __syncthreads();

    // Diagonal 16x16 blocks of T = (I + A)^-1: lane (b, c) solves column c
    // of block b by forward substitution in registers.
    if (w == 0) {
        const int b = l >> 4, c = l & 15;
        const float* Ab = &Am[(16 * b) * LDA + 16 * b];
        float t[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) t[r] = (r == c) ? 1.f : 0.f;
#pragma unroll
        for (int r = 1; r < 16; ++r) {
            float acc = 0.f;
#pragma unroll
            for (int s = 0; s < r; ++s) acc += Ab[r * LDA + s] * t[s];
            if (r > c) t[r] = -acc;
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) Tm[(16 * b + r) * LDA + 16 * b + c] = t[r];
    }
    __syncthreads();

    // Off-diagonal blocks by distance: T_ij = -T_ii * sum_{m=j}^{i-1} A_im T_mj.
    for (int dist = 1; dist < 4; ++dist) {
        const int nblk = 4 - dist;
        if (w < nblk) {
            const int j = w, i = w + dist;
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
            for (int m = j; m < i; ++m)
                acc = mm16_f32(&Am[(16 * i) * LDA + 16 * m], LDA, &Tm[(16 * m) * LDA + 16 * j], LDA, acc, l);
#pragma unroll
            for (int vv = 0; vv < 4; ++vv) Yt[w * 16 * LDY + (4 * (l >> 4) + vv) * LDY + (l & 15)] = acc[vv];
        }
        __syncthreads();
        if (w < nblk) {
            const int j = w, i = w + dist;
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
            acc = mm16_f32(&Tm[(16 * i) * LDA + 16 * i], LDA, &Yt[w * 16 * LDY], LDY, acc, l);
#pragma unroll
            for (int vv = 0; vv < 4; ++vv)
                Tm[(16 * i + 4 * (l >> 4) + vv) * LDA + 16 * j + (l & 15)] = -acc[vv];
        }
        __syncthreads();
    }

    // Power-of-two scales that put T and P into fp16 range:
    // T' = 2^-eT T with max|T'| in [1, 2) (eT >= 0, the diagonal is 1) and
    // P' = 2^-eP P with max|P'| in [2^13, 2^14).  Exact in fp32.
    {
        float mt = 0.f, mp = 0.f;
        for (int it = tid; it < 64 * 64; it += 256) {
            const int r = it >> 6, c = it & 63;
            mt = fmaxf(mt, fabsf(Tm[r * LDA + c]));
            mp = fmaxf(mp, fabsf(Pm[r * LDA + c]));
        }
        mt = wave_max(mt);
        mp = wave_max(mp);
        if (l == 0) {
            red[0][w] = mt;
            red[1][w] = mp;
        }
    }
    __syncthreads();
    const float mt = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
    const float mp = fmaxf(fmaxf(red[1][0], red[1][1]), fmaxf(red[1][2], red[1][3]));
    const int eT = max(0, ilog2f(mt));
    const int eP = mp > 0.f ? min(max(ilog2f(mp) - 13, -kMaxScaleExp), kMaxScaleExp) : 0;
    const float sT = exp2i(-eT), sP = exp2i(-eP);

    // T' and P' (fp16) to the workspace in 32x32x16 A-fragment order:
    // fragment f = 4*mb + ks, lane L holds row 32*mb + L%32, columns
    // 16*ks + 8*(L/32) .. +7.
    const long slot_h = (long)slot * H + h;
    uint8_t* dst = p.tp + slot_h * kSlotBytes;
    for (int it = tid; it < 1024; it += 256) {
        const int mat = it >> 9, f = (it >> 6) & 7, lane = it & 63;
        const int mb = f >> 2, ks = f & 3;
        const int row = 32 * mb + (lane & 31), col = 16 * ks + 8 * (lane >> 5);
        const float* src = mat == 0 ? &Tm[row * LDA + col] : &Pm[row * LDA + col];
        const float sc = mat == 0 ? sT : sP;
        uint4 u;
        u.x = pack_f16x2(src[0] * sc, src[1] * sc);
        u.y = pack_f16x2(src[2] * sc, src[3] * sc);
        u.z = pack_f16x2(src[4] * sc, src[5] * sc);
        u.w = pack_f16x2(src[6] * sc, src[7] * sc);
        *reinterpret_cast<uint4*>(dst + mat * kFragBytes + (f * 64 + lane) * 16) = u;
    }
    if (tid == 0) p.scales[slot_h] = make_int2(eT, eP);
}

// Scan workgroup -> (unit = seq-order index * H + h, tile).  Consecutive
// workgroup ids go round-robin to the 8 XCDs, so the tiles of one unit are
// placed 8 ids apart and share that XCD's L2 (K, Q and T/P are read by every
// tile of the unit).
__device__ __forceinline__ void map_scan_block(int bid, int units, int nt, int& unit, int& tile) {
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

// Registers holding one chunk's inputs while the previous chunk computes.
template <int DK>
struct ChunkRegs {
    uint4 kv[DK / 32], qv[DK / 32];  // K and Q rows, 16-byte pieces
    uint4 vv;                        // 8 values of the V tile
    uint4 frag[4];                   // T' (waves 0,1) or P' (waves 2,3) fp16 fragments
    int2 sc;                         // (eT, eP) of the chunk
    float g, b;                      // wave 0: token lane's log-decay and beta
};

// --------------------------------------------------------------- chunk scan
// Grid: units * n_tiles, 256 threads.  Wave w < DK/32 owns key columns
// [32w, 32w+32) of the workgroup's 32 state rows as one 32x32 fp32 MFMA
// accumulator holding S^T (m = key column, n = state row).
//
// Operand precision: every GEMM runs on fp16 MFMA (11-bit significands)
// with fp32 accumulation; the carried state is fp32.  K and Q are the bf16
// inputs converted exactly to fp16 (L2-normalised rows, |x| <= sqrt(d_k));
// S0, R, U and Uhat are rescaled by one power of two per chunk (eS from the
// state's max over the tile, eR from max|R|) so they stay in fp16 range, and
// the scale is undone exactly in fp32.
template <int DK>
__global__ __launch_bounds__(256) void gdr_chunk_scan_kernel(ChunkParams p) {
    constexpr int LDK = DK + 8;
    constexpr int LDU = 64 + 8;
    constexpr int NSW = DK / 32;  // waves holding state columns
    constexpr int PPR = DK / 8;   // 16-byte pieces per K/Q row
    __shared__ __align__(16) uint16_t Ks[64 * LDK];
    __shared__ __align__(16) uint16_t Qs[64 * LDK];
    __shared__ __align__(16) uint16_t S0s[kTV * LDK];
    __shared__ __align__(16) uint16_t Rt[kTV * LDU];
    __shared__ __align__(16) uint16_t Ut[kTV * LDU];
    __shared__ __align__(16) uint16_t Uh[kTV * LDU];
    __shared__ float Vs[64 * 33];
    __shared__ float Gam[64], Gdl[64], Bs[64];
    __shared__ float Rmx[2];
    __shared__ float Smx[4];

    const int H = p.heads;
    int unit, tile;
    map_scan_block(blockIdx.x, p.batch * H, p.n_tiles, unit, tile);
    const int seqi = unit / H, h = unit - seqi * H;
    const int seq = p.order ? p.order[seqi] : seqi;
    int tb, te;
    seq_bounds(p.cu_seqlens, seq, p.seq_len, tb, te);
    const long slot0 = p.chunk_offsets ? (long)p.chunk_offsets[seq] : (long)seq * p.n_chunks_dense;
    // Overlapping (non-monotonic) cu_seqlens can ask for more chunks than the
    // workspace holds; such input gives unspecified results but every slot
    // index stays inside the workspace.
    const int nch = (int)min((long)(te - tb + kChunk - 1) / kChunk, max(0L, p.n_slots - slot0));
    const int i0 = tile * kTV;
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, ln = l & 31, g2 = l >> 5;
    const int dk = p.d_k, dv = p.d_v;

    // State accumulator: Sacc[4*q4 + e] = S[i0 + ln][32w + 8*q4 + 4*g2 + e].
    f32x16 Sacc;
#pragma unroll
    for (int v = 0; v < 16; ++v) Sacc[v] = 0.f;
    const long sbase = ((long)seq * H + h) * dv * dk;
    if (w < NSW && p.init && i0 + ln < dv) {
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
            const int j = 32 * w + 8 * q4 + 4 * g2;
            if (j < dk) {
                const float4 f = *reinterpret_cast<const float4*>(p.init + sbase + (long)(i0 + ln) * dk + j);
                Sacc[4 * q4 + 0] = f.x;
                Sacc[4 * q4 + 1] = f.y;
                Sacc[4 * q4 + 2] = f.z;
                Sacc[4 * q4 + 3] = f.w;
            }
        }
    }

    // max|S| over the tile, per state-holding wave, for the S0 scale.
    auto state_max = [&]() {
        float m = 0.f;
#pragma unroll
        for (int v = 0; v < 16; ++v) m = fmaxf(m, fabsf(Sacc[v]));
        m = wave_max(m);
        if (l == 0) Smx[w] = m;
    };
    if (w < NSW) state_max();
    __syncthreads();

    ChunkRegs<DK> nx;
    auto fetch = [&](int c) {
        const int t0 = tb + c * kChunk, len = min(kChunk, te - t0);
#pragma unroll
        for (int u = 0; u < DK / 32; ++u) {
            const int it = tid + 256 * u, r = it / PPR, c8 = (it % PPR) * 8;
            uint4 kv = make_uint4(0, 0, 0, 0), qv = make_uint4(0, 0, 0, 0);
            if (r < len && c8 < dk) {
                const long off = ((long)(t0 + r) * H + h) * dk + c8;
                kv = *reinterpret_cast<const uint4*>(p.k + off);
                qv = *reinterpret_cast<const uint4*>(p.q + off);
            }
            nx.kv[u] = kv;
            nx.qv[u] = qv;
        }
        {
            const int r = tid >> 2, c8 = (tid & 3) * 8;
            uint4 vv = make_uint4(0, 0, 0, 0);
            if (r < len && i0 + c8 < dv) vv = *reinterpret_cast<const uint4*>(p.v + ((long)(t0 + r) * H + h) * dv + i0 + c8);
            nx.vv = vv;
        }
        const long slot_h = (slot0 + c) * H + h;
        const uint8_t* src = p.tp + slot_h * kSlotBytes + (w >> 1) * kFragBytes;
        const int mb = w & 1;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
            nx.frag[ks] = *reinterpret_cast<const uint4*>(src + ((mb * 4 + ks) * 64 + l) * 16);
        nx.sc = p.scales[slot_h];
        if (w == 0) {
            float gg = 0.f, bb = 0.f;
            if (l < len) {
                const long gi = (long)(t0 + l) * H + h;
                gg = log_decay(p.gate[gi], p.gate_is_alpha);
                bb = p.beta[gi];
            }
            nx.g = gg;
            nx.b = bb;
        }
    };

    if (nch > 0) fetch(0);
    for (int c = 0; c < nch; ++c) {
        const int t0 = tb + c * kChunk, len = min(kChunk, te - t0);
        // Stage chunk c into LDS, the entering state (bf16) into S0s.
#pragma unroll
        for (int u = 0; u < DK / 32; ++u) {
            const int it = tid + 256 * u, r = it / PPR, c8 = (it % PPR) * 8;
            *reinterpret_cast<uint4*>(&Ks[r * LDK + c8]) = bf16x8_to_f16x8(nx.kv[u]);
            *reinterpret_cast<uint4*>(&Qs[r * LDK + c8]) = bf16x8_to_f16x8(nx.qv[u]);
        }
        {
            const int r = tid >> 2, c8 = (tid & 3) * 8;
            const uint32_t wv[4] = {nx.vv.x, nx.vv.y, nx.vv.z, nx.vv.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                Vs[r * 33 + c8 + 2 * e] = __uint_as_float(wv[e] << 16);
                Vs[r * 33 + c8 + 2 * e + 1] = __uint_as_float(wv[e] & 0xffff0000u);
            }
        }
        f16x8 frag[4];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) frag[ks] = __builtin_bit_cast(f16x8, nx.frag[ks]);
        const int eT = nx.sc.x, eP = nx.sc.y;
        if (w == 0) {
            const float G = chunk_cumsum(nx.g, l);
            const float Glast = __shfl(G, 63, kWave);
            Gam[l] = __expf(G);
            Gdl[l] = __expf(Glast - G);
            Bs[l] = nx.b;
        }
        // S0' = 2^-eS S0 with max|S0'| in [2^14, 2^15).
        float smax = Smx[0];
#pragma unroll
        for (int q = 1; q < NSW; ++q) smax = fmaxf(smax, Smx[q]);
        const int eS = smax > 0.f ? min(max(ilog2f(smax) - 14, -kMaxScaleExp), kMaxScaleExp) : 0;
        if (w < NSW) {
            const float sS = exp2i(-eS);
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                const int j = 32 * w + 8 * q4 + 4 * g2;
                uint2 pk;
                pk.x = pack_f16x2(Sacc[4 * q4 + 0] * sS, Sacc[4 * q4 + 1] * sS);
                pk.y = pack_f16x2(Sacc[4 * q4 + 2] * sS, Sacc[4 * q4 + 3] * sS);
                *reinterpret_cast<uint2*>(&S0s[ln * LDK + j]) = pk;
            }
        }
        if (c + 1 < nch) fetch(c + 1);
        __syncthreads();

        // X = [K; Q] S0^T: wave w takes rows 32*(w&1).. of K (w < 2) or Q.
        const int m0 = 32 * (w & 1);
        f32x16 X;
#pragma unroll
        for (int v = 0; v < 16; ++v) X[v] = 0.f;
        {
            const uint16_t* src = (w < 2) ? Ks : Qs;
#pragma unroll
            for (int kb = 0; kb < DK / 16; ++kb) {
                const f16x8 a = ld_f16x8(&src[(m0 + ln) * LDK + 16 * kb + 8 * g2]);
                const f16x8 b = ld_f16x8(&S0s[ln * LDK + 16 * kb + 8 * g2]);
                X = mfma32h(a, b, X);
            }
            const float up = exp2i(eS);
#pragma unroll
            for (int v = 0; v < 16; ++v) X[v] *= up;
        }
        // X[4*q4+e] is row m0 + 8*q4 + 4*g2 + e (token), column ln (state row).
        // Waves 0,1: R = beta (V - gamma X_K), kept in X; waves 2,3: gamma X_Q.
        if (w < 2) {
            float rm = 0.f;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int s = m0 + 8 * (v >> 2) + 4 * g2 + (v & 3);
                X[v] = Bs[s] * (Vs[s * 33 + ln] - Gam[s] * X[v]);
                rm = fmaxf(rm, fabsf(X[v]));
            }
            rm = wave_max(rm);
            if (l == 0) Rmx[w] = rm;
        } else {
#pragma unroll
            for (int v = 0; v < 16; ++v) X[v] *= Gam[m0 + 8 * (v >> 2) + 4 * g2 + (v & 3)];
        }
        __syncthreads();
        // U = 2^eU U' with R' = 2^-eR R (max|R'| in [2^7, 2^8)), U' = T' R'.
        const float rmax = fmaxf(Rmx[0], Rmx[1]);
        const int eR = rmax > 0.f ? min(max(ilog2f(rmax) - 7, -kMaxScaleExp), kMaxScaleExp) : 0;
        const int eU = eT + eR;
        if (w < 2) {
            const float sR = exp2i(-eR);
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                const int s0 = m0 + 8 * q4 + 4 * g2;
                uint2 pk;
                pk.x = pack_f16x2(X[4 * q4 + 0] * sR, X[4 * q4 + 1] * sR);
                pk.y = pack_f16x2(X[4 * q4 + 2] * sR, X[4 * q4 + 3] * sR);
                *reinterpret_cast<uint2*>(&Rt[ln * LDU + s0]) = pk;
            }
        }
        __syncthreads();

        // U' = T' R' (waves 0, 1: rows 32w..32w+31), stored transposed in
        // fp16, plain (for P U) and scaled by exp(G_last - G_r) (for the
        // state update).  |U'| < 64 * 2 * 2^8, inside fp16 range.
        if (w < 2) {
            f32x16 U;
#pragma unroll
            for (int v = 0; v < 16; ++v) U[v] = 0.f;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) U = mfma32h(frag[ks], ld_f16x8(&Rt[ln * LDU + 16 * ks + 8 * g2]), U);
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                const int r0 = 32 * w + 8 * q4 + 4 * g2;
                uint2 pk;
                pk.x = pack_f16x2(U[4 * q4 + 0], U[4 * q4 + 1]);
                pk.y = pack_f16x2(U[4 * q4 + 2], U[4 * q4 + 3]);
                *reinterpret_cast<uint2*>(&Ut[ln * LDU + r0]) = pk;
                pk.x = pack_f16x2(Gdl[r0 + 0] * U[4 * q4 + 0], Gdl[r0 + 1] * U[4 * q4 + 1]);
                pk.y = pack_f16x2(Gdl[r0 + 2] * U[4 * q4 + 2], Gdl[r0 + 3] * U[4 * q4 + 3]);
                *reinterpret_cast<uint2*>(&Uh[ln * LDU + r0]) = pk;
            }
        }
        __syncthreads();

        // O = gamma Q S0^T + 2^(eP+eU) P' U' (waves 2, 3), stored as bf16.
        if (w >= 2) {
            const int eO = eP + eU;
            const float down = exp2i(-eO), up = exp2i(eO);
#pragma unroll
            for (int v = 0; v < 16; ++v) X[v] *= down;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) X = mfma32h(frag[ks], ld_f16x8(&Ut[ln * LDU + 16 * ks + 8 * g2]), X);
            const int i = i0 + ln;
            if (i < dv) {
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int r = m0 + 8 * (v >> 2) + 4 * g2 + (v & 3);
                    if (r < len) p.o[((long)(t0 + r) * H + h) * dv + i] = f32_to_bf16(X[v] * up);
                }
            }
        }
        // S^T <- gamma_last S^T + 2^eU K^T Uhat' (waves holding state columns).
        if (w < NSW) {
            const float down = Gam[63] * exp2i(-eU), up = exp2i(eU);
#pragma unroll
            for (int v = 0; v < 16; ++v) Sacc[v] *= down;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const uint16_t* kc = &Ks[(16 * ks + 8 * g2) * LDK + 32 * w + ln];
                uint4 u;
                u.x = uint32_t(kc[0 * LDK]) | (uint32_t(kc[1 * LDK]) << 16);
                u.y = uint32_t(kc[2 * LDK]) | (uint32_t(kc[3 * LDK]) << 16);
                u.z = uint32_t(kc[4 * LDK]) | (uint32_t(kc[5 * LDK]) << 16);
                u.w = uint32_t(kc[6 * LDK]) | (uint32_t(kc[7 * LDK]) << 16);
                Sacc = mfma32h(__builtin_bit_cast(f16x8, u), ld_f16x8(&Uh[ln * LDU + 16 * ks + 8 * g2]), Sacc);
            }
#pragma unroll
            for (int v = 0; v < 16; ++v) Sacc[v] *= up;
            state_max();
        }
        __syncthreads();
    }

    if (p.fin && w < NSW && i0 + ln < dv) {
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
            const int j = 32 * w + 8 * q4 + 4 * g2;
            if (j < dk)
                *reinterpret_cast<float4*>(p.fin + sbase + (long)(i0 + ln) * dk + j) =
                    make_float4(Sacc[4 * q4 + 0], Sacc[4 * q4 + 1], Sacc[4 * q4 + 2], Sacc[4 * q4 + 3]);
        }
    }
}

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

struct WsLayout {
    size_t offsets, order, scales, tp, total;
    long n_slots;
};

WsLayout ws_layout(const rhz_gdr_prefill_args& a) {
    WsLayout L;
    const long n = a.batch;
    if (a.cu_seqlens) L.n_slots = ((long)a.seq_len + kChunk - 1) / kChunk + n;
    else L.n_slots = n * (((long)a.seq_len + kChunk - 1) / kChunk);
    L.offsets = 0;
    L.order = align256(sizeof(int) * (n + 1));
    L.scales = L.order + align256(sizeof(int) * n);
    L.tp = L.scales + align256(sizeof(int2) * (size_t)L.n_slots * a.heads);
    L.total = L.tp + (size_t)L.n_slots * a.heads * kSlotBytes;
    return L;
}

template <int DK>
hipError_t chunked_go(const ChunkParams& cp, long n_slots, int heads, int units_x_tiles, hipStream_t st) {
    if (n_slots > 0)
        hipLaunchKernelGGL(gdr_chunk_prep_kernel<DK>, dim3((unsigned)n_slots, heads), dim3(256), 0, st, cp);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(gdr_chunk_scan_kernel<DK>, dim3(units_x_tiles), dim3(256), 0, st, cp);
    return hipGetLastError();
}

}  // namespace

bool chunked_supported(int d_k, int d_v) {
    return d_k >= 8 && d_k <= 128 && d_k % 8 == 0 && d_v >= 8 && d_v % 8 == 0;
}

size_t chunked_workspace_bytes(const rhz_gdr_prefill_args& a) { return ws_layout(a).total; }

hipError_t launch_chunked(const rhz_gdr_prefill_args& a, hipStream_t st) {
    const WsLayout L = ws_layout(a);
    uint8_t* ws = static_cast<uint8_t*>(a.workspace);
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
    cp.tp = ws + L.tp;
    cp.scales = reinterpret_cast<int2*>(ws + L.scales);
    cp.batch = a.batch;
    cp.seq_len = a.seq_len;
    cp.heads = a.heads;
    cp.d_k = a.d_k;
    cp.d_v = a.d_v;
    cp.gate_is_alpha = a.gate_kind == RHZ_GATE_ALPHA;
    cp.n_chunks_dense = (a.seq_len + kChunk - 1) / kChunk;
    cp.n_tiles = (a.d_v + kTV - 1) / kTV;
    cp.n_slots = L.n_slots;
    if (a.cu_seqlens) {
        int* offsets = reinterpret_cast<int*>(ws + L.offsets);
        int* order = reinterpret_cast<int*>(ws + L.order);
        hipLaunchKernelGGL(gdr_varlen_setup_kernel, dim3(1), dim3(1024), 0, st, a.cu_seqlens, a.batch,
                           a.seq_len, offsets, order);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        cp.chunk_offsets = offsets;
        cp.order = order;
    } else {
        cp.chunk_offsets = nullptr;
        cp.order = nullptr;
    }
    const int units_x_tiles = a.batch * a.heads * cp.n_tiles;
    if (a.d_k <= 64) return chunked_go<64>(cp, L.n_slots, a.heads, units_x_tiles, st);
    return chunked_go<128>(cp, L.n_slots, a.heads, units_x_tiles, st);
}

}  // namespace rhz
