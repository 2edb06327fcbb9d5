// gdr_device.hpp -- device helpers shared by the gfx950 gated delta-rule kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rhz {

// Vector types of the gfx950 MFMA builtins.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// Chunk length of the WY/UT prefill and its reset threshold: a token whose
// log-decay is at or below kLogDecayFloor (alpha <= 1.8e-35, including
// alpha = 0) starts a new segment inside its chunk -- everything before it is
// forgotten exactly, as a reset does in the reference (delta.rs:137-142) --
// and every other log-decay enters the chunk's prefix sums unchanged.
constexpr int kChunk = 64;
constexpr float kLogDecayFloor = -80.0f;

__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float(uint32_t(h) << 16); }

// float -> bf16, round to nearest even (NaN stays NaN).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return uint16_t(u >> 16);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    return uint32_t(f32_to_bf16(lo)) | (uint32_t(f32_to_bf16(hi)) << 16);
}

// float -> fp16 bits, round to nearest even.
__device__ __forceinline__ uint16_t f32_to_f16(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
    return uint32_t(f32_to_f16(lo)) | (uint32_t(f32_to_f16(hi)) << 16);
}

// 2^e as a float, e clamped to the normal range [-126, 127].
__device__ __forceinline__ float exp2i(int e) {
    e = min(max(e, -126), 127);
    return __int_as_float((e + 127) << 23);
}

// floor(log2(m)) for a positive normal float m (-127 for zero/subnormal).
__device__ __forceinline__ int ilog2f(float m) { return int((__float_as_uint(m) >> 23) & 0xffu) - 127; }

// Cross-lane move within rows of 16 lanes (DPP); lanes without a source read 0.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xf, 0xf, true));
}

// Maximum over the 64 lanes of a wave, returned to every lane: DPP within
// rows of 16 (quad_perm [1,0,3,2], [2,3,0,1], row_ror 4, row_ror 8), then the
// four row maxima through scalar registers.
__device__ __forceinline__ float wave_max(float x) {
    x = fmaxf(x, dpp_mov<0xB1>(x));
    x = fmaxf(x, dpp_mov<0x4E>(x));
    x = fmaxf(x, dpp_mov<0x124>(x));
    x = fmaxf(x, dpp_mov<0x128>(x));
    const int xi = __builtin_bit_cast(int, x);
    const float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(xi, 0));
    const float b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(xi, 16));
    const float c = __builtin_bit_cast(float, __builtin_amdgcn_readlane(xi, 32));
    const float d = __builtin_bit_cast(float, __builtin_amdgcn_readlane(xi, 48));
    return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

// Element loads of the two input dtypes, widened to float.
template <typename T> struct Elem;
template <> struct Elem<float> {
    static __device__ __forceinline__ float load(const float* p, long i) { return p[i]; }
    static __device__ __forceinline__ void store(float* p, long i, float x) { p[i] = x; }
};
template <> struct Elem<uint16_t> {
    static __device__ __forceinline__ float load(const uint16_t* p, long i) { return bf16_to_f32(p[i]); }
    static __device__ __forceinline__ void store(uint16_t* p, long i, float x) { p[i] = f32_to_bf16(x); }
};

// Four consecutive elements widened to float (caller guarantees alignment:
// 16 bytes for float, 8 bytes for bf16).
__device__ __forceinline__ float4 load4(const float* p) { return *reinterpret_cast<const float4*>(p); }
__device__ __forceinline__ float4 load4(const uint16_t* p) {
    uint2 u = *reinterpret_cast<const uint2*>(p);
    return make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u),
                       __uint_as_float(u.y << 16), __uint_as_float(u.y & 0xffff0000u));
}

// Sum over aligned groups of G consecutive lanes (G a power of two <= 64);
// every lane of the group receives the group's sum.  Fixed butterfly order,
// so the result is deterministic.
template <int G>
__device__ __forceinline__ float group_sum(float x) {
#pragma unroll
    for (int off = G / 2; off >= 1; off >>= 1) x += __shfl_xor(x, off, kWave);
    return x;
}

// Sum over aligned groups of G (2, 4, 8 or 16) lanes by DPP within rows of
// 16: quad_perm [1,0,3,2], [2,3,0,1], then row_half_mirror and row_mirror.
// The pairings are symmetric, so every lane of a group gets the same bits.
template <int G>
__device__ __forceinline__ float lane_group_sum(float x) {
    static_assert(G == 2 || G == 4 || G == 8 || G == 16, "group of 2, 4, 8 or 16 lanes");
    x += dpp_mov<0xB1>(x);
    if constexpr (G >= 4) x += dpp_mov<0x4E>(x);
    if constexpr (G >= 8) x += dpp_mov<0x141>(x);
    if constexpr (G >= 16) x += dpp_mov<0x140>(x);
    return x;
}

// Token range [t0, t1) of sequence `seq`: packed through cu (clamped into
// [0, total]) or dense with seq_len tokens each.
__device__ __forceinline__ void seq_bounds(const int* cu, int seq, int seq_len, int& t0, int& t1) {
    if (cu) {
        t0 = min(max(cu[seq], 0), seq_len);
        t1 = min(max(cu[seq + 1], t0), seq_len);
    } else {
        t0 = seq * seq_len;
        t1 = t0 + seq_len;
    }
}

// Gate value -> log-decay g (<= 0 expected; -inf for alpha = 0).
__device__ __forceinline__ float log_decay(float gate, int gate_is_alpha) {
    return gate_is_alpha ? logf(gate) : gate;
}

// Whether a log-decay resets the state (at or below kLogDecayFloor; a NaN
// gate is no reset and carries into the outputs, as in the recurrence).
__device__ __forceinline__ bool is_reset(float g) { return g <= kLogDecayFloor; }

// The prologue's elementwise maps (elementwise.rs:5-12, 36-42).
__device__ __forceinline__ float sigmoid_f(float x) {
    if (x >= 0.f) return 1.f / (1.f + expf(-x));
    const float e = expf(x);
    return e / (1.f + e);
}
__device__ __forceinline__ float softplus_f(float x) { return x > 30.f ? x : log1pf(expf(x)); }

// Gate value -> alpha.
__device__ __forceinline__ float decay_factor(float gate, int gate_is_alpha) {
    return gate_is_alpha ? gate : expf(gate);
}

}  // namespace rhz
