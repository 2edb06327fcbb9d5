// gdr_philox.hip -- seeded synthetic inputs on the device from the
// reference's counter-based Philox-4x32-10 (crates/ops/src/rng.rs:7-90):
// element e takes normal #e of stream (seed, stream_id), i.e. the
// Box-Muller (cosine branch) pair of Philox block e, in f64, then the
// elementwise transforms of crates/ops/src/elementwise.rs (sigmoid 5-12,
// softplus 36-42, l2norm 125-128) before rounding to the output dtype.

#include "gdr_device.hpp"
#include "gdr_internal.hpp"

namespace rhz {
namespace {

__device__ __forceinline__ void philox_block(uint64_t seed, uint64_t stream, uint64_t counter,
                                             uint32_t out[4]) {
    uint32_t c0 = uint32_t(counter), c1 = uint32_t(counter >> 32);
    uint32_t c2 = uint32_t(stream), c3 = uint32_t(stream >> 32);
    uint32_t k0 = uint32_t(seed >> 32), k1 = uint32_t(seed);
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        const uint64_t p0 = uint64_t(c0) * 0xD2511F53u;
        const uint64_t p1 = uint64_t(c2) * 0xCD9E8D57u;
        const uint32_t n0 = uint32_t(p1 >> 32) ^ c1 ^ k0;
        const uint32_t n2 = uint32_t(p0 >> 32) ^ c3 ^ k1;
        c1 = uint32_t(p1);
        c3 = uint32_t(p0);
        c0 = n0;
        c2 = n2;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    out[0] = c0;
    out[1] = c1;
    out[2] = c2;
    out[3] = c3;
}

// rng.rs:78-90 applied to one aligned block.
__device__ __forceinline__ double philox_normal(uint64_t seed, uint64_t stream, uint64_t idx) {
    uint32_t b[4];
    philox_block(seed, stream, idx, b);
    const double two53 = 9007199254740992.0;
    double u1 = double((uint64_t(b[0] >> 5) << 26) | uint64_t(b[1] >> 6)) / two53;
    const double u2 = double((uint64_t(b[2] >> 5) << 26) | uint64_t(b[3] >> 6)) / two53;
    if (u1 < 1e-300) u1 = 1e-300;
    return sqrt(-2.0 * log(u1)) * cos(6.28318530717958647692528676655900577 * u2);
}

// rng.rs:78-82 on u32 words 2e and 2e + 1 of the stream: next_f64 #e.
__device__ __forceinline__ double philox_uniform(uint64_t seed, uint64_t stream, uint64_t e) {
    uint32_t b[4];
    philox_block(seed, stream, e >> 1, b);
    const uint32_t w0 = (e & 1) ? b[2] : b[0], w1 = (e & 1) ? b[3] : b[1];
    return double((uint64_t(w0 >> 5) << 26) | uint64_t(w1 >> 6)) / 9007199254740992.0;
}

__device__ __forceinline__ double sigmoid_f64(double x) {
    if (x >= 0.0) return 1.0 / (1.0 + exp(-x));
    const double e = exp(x);
    return e / (1.0 + e);
}

__device__ __forceinline__ double softplus_f64(double x) { return x > 30.0 ? x : log(1.0 + exp(x)); }

__device__ __forceinline__ void put(void* out, int dtype, int64_t i, double x) {
    if (dtype == 2) {
        static_cast<double*>(out)[i] = x;
    } else if (dtype == RHZ_F32) {
        static_cast<float*>(out)[i] = float(x);
    } else {
        static_cast<uint16_t*>(out)[i] = f32_to_bf16(float(x));
    }
}

__global__ __launch_bounds__(256) void philox_fill_kernel(int kind, uint64_t seed, uint64_t sid,
                                                          int64_t count, double mean, double sd,
                                                          int dtype, void* out) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= count) return;
    if (kind == RHZ_FILL_UNIFORM) {
        put(out, dtype, i, philox_uniform(seed, sid, uint64_t(i)));
        return;
    }
    const double z = philox_normal(seed, sid, uint64_t(i));
    const double x = (mean == 0.0 && sd == 1.0) ? z : mean + sd * z;
    double y = x;
    if (kind == RHZ_FILL_SIGMOID) y = sigmoid_f64(x);
    else if (kind == RHZ_FILL_NEG_SOFTPLUS) y = -softplus_f64(x);
    put(out, dtype, i, y);
}

// One thread per row: the sum of squares in element order (as
// elementwise.rs:126), then z / n * 1.0 with n floored at 1e-12.
__global__ __launch_bounds__(256) void philox_unit_rows_kernel(uint64_t seed, uint64_t sid, int64_t rows,
                                                               int row_len, int dtype, void* out) {
    const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (r >= rows) return;
    const int64_t e0 = r * row_len;
    double ss = 0.0;
    for (int j = 0; j < row_len; ++j) {
        const double z = philox_normal(seed, sid, uint64_t(e0 + j));
        ss += z * z;
    }
    double n = sqrt(ss);
    if (n < 1e-12) n = 1e-12;
    for (int j = 0; j < row_len; ++j) {
        const double z = philox_normal(seed, sid, uint64_t(e0 + j));
        put(out, dtype, e0 + j, z / n * 1.0);
    }
}

}  // namespace

hipError_t launch_philox_fill(int kind, uint64_t seed, uint64_t sid, int64_t count, int row_len, double mean,
                              double sd, int dtype, void* out, hipStream_t st) {
    if (count <= 0) return hipSuccess;
    if (kind == RHZ_FILL_UNIT_ROWS) {
        const int64_t rows = count / row_len;
        hipLaunchKernelGGL(philox_unit_rows_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, st, seed,
                           sid, rows, row_len, dtype, out);
    } else {
        hipLaunchKernelGGL(philox_fill_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, st, kind, seed,
                           sid, count, mean, sd, dtype, out);
    }
    return hipGetLastError();
}

}  // namespace rhz
