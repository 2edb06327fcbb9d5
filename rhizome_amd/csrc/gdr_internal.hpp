// gdr_internal.hpp -- host-side launch interface between the C ABI layer
// (gdr_abi.cpp) and the kernel files.  Arguments are validated by the
// caller before any of these run.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "rhizome_gdr.h"

namespace rhz {

// Token-sequential fp32 recurrence over a dense or packed batch.
hipError_t launch_recurrent(const rhz_gdr_prefill_args& a, hipStream_t stream);

// One decode position for every (b, h), state in place.
hipError_t launch_decode(const rhz_gdr_decode_args& a, hipStream_t stream);

// Up to RHZ_MULTISTEP_MAX positions for every (b, h), with per-position
// state snapshots.
hipError_t launch_multistep(const rhz_gdr_multistep_args& a, hipStream_t stream);

// Chunked WY/UT prefill (bf16 in, fp32 state).  Requires d_k % 8 == 0,
// d_k <= 128, d_v % 8 == 0 and 16-byte aligned tensors.
bool chunked_supported(int d_k, int d_v);
size_t chunked_workspace_bytes(const rhz_gdr_prefill_args& a);
// The fused prologue of rhz_gdr_local_prefill: a.q and a.k are the raw
// projections, a.gate holds alpha logits and a.beta beta logits.
struct ChunkPrologue {
    const float* a_log;  // [H]
    float q_scale;
};
// spin_limit: polls after which an LDS wait gives up; <= 0 for the built-in
// limit (tests pass a tiny one to force give-ups).  pro: the fused prologue,
// or nullptr.
hipError_t launch_chunked(const rhz_gdr_prefill_args& a, hipStream_t stream, int spin_limit = 0,
                          const ChunkPrologue* pro = nullptr);
// The chunked launch of rhz_gdr_prefill_noalloc: the packed-batch order
// lives in a static device array of kNoAllocMaxSeqs ints (a.workspace is
// not used); the caller has checked a.batch <= kNoAllocMaxSeqs for packed
// batches.
constexpr int kNoAllocMaxSeqs = RHZ_NOALLOC_MAX_SEQS;
hipError_t launch_chunked_noalloc(const rhz_gdr_prefill_args& a, hipStream_t stream);
// Reads (and with `reset`, zeroes) the current device's count of chunked-kernel
// LDS waits that gave up.  Synchronous with respect to the device.
hipError_t chunked_sync_timeouts(unsigned int* count, bool reset);
// The same for the count of (workgroup, wave) pairs of the fused-prologue
// instances that saw an fp16 operand that was not finite or beyond fp16's
// range.
hipError_t chunked_range_errors(unsigned int* count, bool reset);
// The same for the count of workgroups that recomputed their rows with the
// fp32 recurrence because an input left the fp16 path's domain.
hipError_t chunked_exact_reruns(unsigned int* count, bool reset);

// Local-block prologue and epilogue (gdr_aux.hip).
hipError_t launch_conv1d(const rhz_conv1d_args& a, hipStream_t stream);
hipError_t launch_prepare(const rhz_gdr_prepare_args& a, hipStream_t stream);
hipError_t launch_rmsnorm(const rhz_rmsnorm_args& a, hipStream_t stream);
// conv1d and prepare in one pass; the caller has checked
// conv_prepare_supported(dtype, d_k, d_v).
bool conv_prepare_supported(int dtype, int d_k, int d_v);
hipError_t launch_conv_prepare(const rhz_gdr_conv_prepare_args& a, hipStream_t stream);

// Device Philox-4x32-10 fill.
hipError_t launch_philox_fill(int kind, uint64_t seed, uint64_t stream_id, int64_t count,
                              int row_len, double mean, double std_dev, int out_dtype, void* out,
                              hipStream_t stream);

}  // namespace rhz
