// gdr_abi.cpp -- the extern "C" boundary of librhizome_gdr.so: argument
// validation (complete before any HIP call, so every error path can be
// exercised without a GPU), algorithm selection, workspace sizing and
// dispatch to the kernel launchers.

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <string>

#include "gdr_internal.hpp"
#include "rhizome_gdr.h"

namespace {

thread_local std::string g_last_error;

rhz_status fail(rhz_status s, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return s;
}

rhz_status ok() {
    g_last_error.clear();
    return RHZ_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

constexpr int64_t kMaxIndex = INT32_MAX;

// Validates a prefill call and resolves its algorithm.  Pointers are checked
// only when check_ptrs is set (the workspace query reads none).
rhz_status check_prefill(const rhz_gdr_prefill_args* a, bool check_ptrs, int* algo_out) {
    if (!a) return fail(RHZ_ERR_INVALID_ARG, "args is NULL");
    if (a->batch < 1) return fail(RHZ_ERR_INVALID_ARG, "batch must be >= 1 (got %d)", a->batch);
    if (a->seq_len < 0) return fail(RHZ_ERR_INVALID_ARG, "seq_len must be >= 0 (got %d)", a->seq_len);
    if (a->heads < 1) return fail(RHZ_ERR_INVALID_ARG, "heads must be >= 1 (got %d)", a->heads);
    if (a->d_k < 1) return fail(RHZ_ERR_INVALID_ARG, "d_k must be >= 1 (got %d)", a->d_k);
    if (a->d_v < 1) return fail(RHZ_ERR_INVALID_ARG, "d_v must be >= 1 (got %d)", a->d_v);
    if (a->chunk < 1) return fail(RHZ_ERR_INVALID_ARG, "chunk must be >= 1 (got %d)", a->chunk);
    if (a->dtype != RHZ_F32 && a->dtype != RHZ_BF16)
        return fail(RHZ_ERR_INVALID_ARG, "dtype must be RHZ_F32 or RHZ_BF16 (got %d)", a->dtype);
    if (a->gate_kind != RHZ_GATE_LOG_ALPHA && a->gate_kind != RHZ_GATE_ALPHA)
        return fail(RHZ_ERR_INVALID_ARG, "gate_kind must be RHZ_GATE_LOG_ALPHA or RHZ_GATE_ALPHA (got %d)",
                    a->gate_kind);
    if (a->algo < RHZ_ALGO_AUTO || a->algo > RHZ_ALGO_CHUNKED)
        return fail(RHZ_ERR_INVALID_ARG, "algo must be AUTO, RECURRENT or CHUNKED (got %d)", a->algo);
    if (a->d_k > 256) return fail(RHZ_ERR_UNSUPPORTED, "d_k = %d exceeds the supported 256", a->d_k);
    if (a->d_v > 1024) return fail(RHZ_ERR_UNSUPPORTED, "d_v = %d exceeds the supported 1024", a->d_v);
    const int64_t tokens = a->cu_seqlens ? (int64_t)a->seq_len : (int64_t)a->batch * a->seq_len;
    if (tokens * a->heads > kMaxIndex)
        return fail(RHZ_ERR_INVALID_ARG, "tokens * heads = %lld exceeds 2^31 - 1", (long long)(tokens * a->heads));
    const int64_t units = (int64_t)a->batch * a->heads;
    if (units * ((a->d_v + 7) / 8) > kMaxIndex)
        return fail(RHZ_ERR_INVALID_ARG, "batch * heads = %lld is too large", (long long)units);

    int algo = a->algo;
    const bool chunk_dims = rhz::chunked_supported(a->d_k, a->d_v);
    if (algo == RHZ_ALGO_AUTO) algo = (a->dtype == RHZ_BF16 && chunk_dims) ? RHZ_ALGO_CHUNKED : RHZ_ALGO_RECURRENT;
    if (algo == RHZ_ALGO_CHUNKED) {
        if (a->dtype != RHZ_BF16) return fail(RHZ_ERR_UNSUPPORTED, "CHUNKED needs bf16 q/k/v (dtype %d)", a->dtype);
        if (!chunk_dims)
            return fail(RHZ_ERR_UNSUPPORTED,
                        "CHUNKED needs d_k in 8..128 and d_v >= 8, both multiples of 8 (got d_k=%d d_v=%d)",
                        a->d_k, a->d_v);
        // The kernel addresses one 64-token chunk of a head with 32-bit byte offsets.
        if ((int64_t)a->heads * std::max(a->d_k, a->d_v) * 2 * 64 > kMaxIndex)
            return fail(RHZ_ERR_UNSUPPORTED, "CHUNKED needs heads * max(d_k, d_v) below 2^24 (got %lld)",
                        (long long)a->heads * std::max(a->d_k, a->d_v));
    }
    *algo_out = algo;
    if (!check_ptrs) return ok();

    if (tokens > 0) {
        if (!a->q) return fail(RHZ_ERR_INVALID_ARG, "q is NULL");
        if (!a->k) return fail(RHZ_ERR_INVALID_ARG, "k is NULL");
        if (!a->v) return fail(RHZ_ERR_INVALID_ARG, "v is NULL");
        if (!a->gate) return fail(RHZ_ERR_INVALID_ARG, "gate is NULL");
        if (!a->beta) return fail(RHZ_ERR_INVALID_ARG, "beta is NULL");
        if (!a->o) return fail(RHZ_ERR_INVALID_ARG, "o is NULL");
    }
    if (algo == RHZ_ALGO_CHUNKED) {
        const void* ptrs[] = {a->q, a->k, a->v, a->o, a->initial_state, a->final_state};
        const char* names[] = {"q", "k", "v", "o", "initial_state", "final_state"};
        for (int i = 0; i < 6; ++i)
            if (!aligned16(ptrs[i]))
                return fail(RHZ_ERR_INVALID_ARG, "CHUNKED needs %s 16-byte aligned", names[i]);
    } else {
        const size_t ea = a->dtype == RHZ_F32 ? 4 : 2;
        const void* ptrs[] = {a->q, a->k, a->v, a->o};
        const char* names[] = {"q", "k", "v", "o"};
        for (int i = 0; i < 4; ++i)
            if (reinterpret_cast<uintptr_t>(ptrs[i]) % ea)
                return fail(RHZ_ERR_INVALID_ARG, "%s is not aligned to its element size", names[i]);
    }
    if (reinterpret_cast<uintptr_t>(a->gate) % 4 || reinterpret_cast<uintptr_t>(a->beta) % 4 ||
        reinterpret_cast<uintptr_t>(a->initial_state) % 4 || reinterpret_cast<uintptr_t>(a->final_state) % 4 ||
        reinterpret_cast<uintptr_t>(a->cu_seqlens) % 4)
        return fail(RHZ_ERR_INVALID_ARG, "fp32/int32 tensors must be 4-byte aligned");
    return ok();
}

rhz_status hip_status(hipError_t e, const char* what) {
    if (e == hipSuccess) return ok();
    return fail(RHZ_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

}  // namespace

extern "C" {

int32_t rhz_gdr_abi_version(void) { return RHZ_GDR_ABI_VERSION; }

const char* rhz_status_string(int32_t status) {
    switch (status) {
        case RHZ_OK: return "RHZ_OK";
        case RHZ_ERR_INVALID_ARG: return "RHZ_ERR_INVALID_ARG";
        case RHZ_ERR_UNSUPPORTED: return "RHZ_ERR_UNSUPPORTED";
        case RHZ_ERR_WORKSPACE: return "RHZ_ERR_WORKSPACE";
        case RHZ_ERR_HIP: return "RHZ_ERR_HIP";
        default: return "RHZ_ERR_UNKNOWN";
    }
}

const char* rhz_last_error(void) { return g_last_error.c_str(); }

rhz_status rhz_gdr_query_support(int32_t op, int32_t dtype, int32_t d_k, int32_t d_v, int32_t algo) {
    if (op != RHZ_OP_DELTA_SCAN && op != RHZ_OP_DELTA_STEP && op != RHZ_OP_DELTA_MULTISTEP)
        return fail(RHZ_ERR_INVALID_ARG, "unknown op %d", op);
    if (dtype != RHZ_F32 && dtype != RHZ_BF16) return fail(RHZ_ERR_INVALID_ARG, "unknown dtype %d", dtype);
    if (algo < RHZ_ALGO_AUTO || algo > RHZ_ALGO_CHUNKED) return fail(RHZ_ERR_INVALID_ARG, "unknown algo %d", algo);
    if (d_k < 1 || d_v < 1) return fail(RHZ_ERR_INVALID_ARG, "d_k and d_v must be >= 1");
    if (d_k > 256 || d_v > 1024)
        return fail(RHZ_ERR_UNSUPPORTED, "d_k <= 256 and d_v <= 1024 are supported (got %d, %d)", d_k, d_v);
    if (op == RHZ_OP_DELTA_STEP || op == RHZ_OP_DELTA_MULTISTEP) {
        if (algo == RHZ_ALGO_CHUNKED)
            return fail(RHZ_ERR_UNSUPPORTED, "the decode step and multistep have no CHUNKED algorithm");
        return ok();
    }
    if (algo == RHZ_ALGO_CHUNKED) {
        if (dtype != RHZ_BF16) return fail(RHZ_ERR_UNSUPPORTED, "CHUNKED needs bf16 inputs");
        if (!rhz::chunked_supported(d_k, d_v))
            return fail(RHZ_ERR_UNSUPPORTED, "CHUNKED needs d_k in 8..128 and d_v >= 8, multiples of 8");
    }
    return ok();
}

rhz_status rhz_gdr_prefill_workspace_size(const rhz_gdr_prefill_args* args, size_t* bytes) {
    if (!bytes) return fail(RHZ_ERR_INVALID_ARG, "bytes is NULL");
    int algo = 0;
    const rhz_status s = check_prefill(args, false, &algo);
    if (s != RHZ_OK) return s;
    *bytes = algo == RHZ_ALGO_CHUNKED ? rhz::chunked_workspace_bytes(*args) : 0;
    return ok();
}

namespace {
rhz_status prefill_impl(const rhz_gdr_prefill_args* args, void* stream, int spin_limit,
                        const rhz::ChunkPrologue* pro = nullptr);
}  // namespace

rhz_status rhz_gdr_prefill(const rhz_gdr_prefill_args* args, void* stream) { return prefill_impl(args, stream, 0); }

rhz_status rhz_gdr_prefill_spin_limit(const rhz_gdr_prefill_args* args, int32_t spin_limit, void* stream) {
    if (spin_limit < 1) return fail(RHZ_ERR_INVALID_ARG, "spin_limit must be >= 1 (got %d)", spin_limit);
    return prefill_impl(args, stream, spin_limit);
}

rhz_status rhz_gdr_prefill_noalloc(const rhz_gdr_prefill_args* args, void* stream) {
    int algo = 0;
    const rhz_status s = check_prefill(args, true, &algo);
    if (s != RHZ_OK) return s;
    if (args->seq_len == 0 && !args->final_state) return ok();
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (algo == RHZ_ALGO_CHUNKED) {
        if (args->cu_seqlens && args->batch > RHZ_NOALLOC_MAX_SEQS)
            return fail(RHZ_ERR_UNSUPPORTED, "rhz_gdr_prefill_noalloc takes at most %d packed sequences (got %d)",
                        RHZ_NOALLOC_MAX_SEQS, args->batch);
        return hip_status(rhz::launch_chunked_noalloc(*args, st), "chunked prefill launch (no allocation)");
    }
    return hip_status(rhz::launch_recurrent(*args, st), "recurrent prefill launch");
}

rhz_status rhz_gdr_local_prefill(const rhz_gdr_local_args* args, void* stream) {
    if (!args) return fail(RHZ_ERR_INVALID_ARG, "args is NULL");
    rhz_gdr_prefill_args a = args->prefill;
    a.gate = args->alpha_logit;
    a.beta = args->beta_logit;
    a.gate_kind = RHZ_GATE_LOG_ALPHA;
    int algo = 0;
    rhz_status s = check_prefill(&a, false, &algo);
    if (s != RHZ_OK) return s;
    if (algo != RHZ_ALGO_CHUNKED)
        return fail(RHZ_ERR_UNSUPPORTED, "the fused prologue runs on the CHUNKED path only (bf16, d_k 8..128)");
    if (!std::isfinite(args->q_scale)) return fail(RHZ_ERR_INVALID_ARG, "q_scale must be finite");
    // the prepared q has elements of at most |q_scale| and q.k products of at
    // most |q_scale| (unit rows), so this bound keeps every fp16 operand the
    // kernel forms from q and k in range whatever the raw projections hold
    if (!(std::fabs(args->q_scale) <= 32768.f))
        return fail(RHZ_ERR_UNSUPPORTED, "|q_scale| above 2^15 would take the chunked kernel's fp16 operands out of "
                                         "range; use rhz_gdr_prepare and RHZ_ALGO_RECURRENT");
    const int64_t tokens = a.cu_seqlens ? (int64_t)a.seq_len : (int64_t)a.batch * a.seq_len;
    if (tokens > 0) {
        if (!args->beta_logit) return fail(RHZ_ERR_INVALID_ARG, "beta_logit is NULL");
        if (!args->alpha_logit) return fail(RHZ_ERR_INVALID_ARG, "alpha_logit is NULL");
        if (!args->a_log) return fail(RHZ_ERR_INVALID_ARG, "a_log is NULL");
    }
    if (reinterpret_cast<uintptr_t>(args->a_log) % 4) return fail(RHZ_ERR_INVALID_ARG, "a_log must be 4-byte aligned");
    const rhz::ChunkPrologue pro{args->a_log, args->q_scale};
    return prefill_impl(&a, stream, 0, &pro);
}

rhz_status rhz_gdr_sync_timeouts(uint32_t* count, int32_t reset) {
    if (!count) return fail(RHZ_ERR_INVALID_ARG, "count is NULL");
    unsigned int n = 0;
    const hipError_t e = rhz::chunked_sync_timeouts(&n, reset != 0);
    if (e != hipSuccess) return hip_status(e, "reading the sync timeout count");
    *count = n;
    return ok();
}

rhz_status rhz_gdr_fp16_range_errors(uint32_t* count, int32_t reset) {
    if (!count) return fail(RHZ_ERR_INVALID_ARG, "count is NULL");
    unsigned int n = 0;
    const hipError_t e = rhz::chunked_range_errors(&n, reset != 0);
    if (e != hipSuccess) return hip_status(e, "reading the fp16 range error count");
    *count = n;
    return ok();
}

rhz_status rhz_gdr_exact_reruns(uint32_t* count, int32_t reset) {
    if (!count) return fail(RHZ_ERR_INVALID_ARG, "count is NULL");
    unsigned int n = 0;
    const hipError_t e = rhz::chunked_exact_reruns(&n, reset != 0);
    if (e != hipSuccess) return hip_status(e, "reading the exact rerun count");
    *count = n;
    return ok();
}

}  // extern "C"

namespace {
rhz_status prefill_impl(const rhz_gdr_prefill_args* args, void* stream, int spin_limit,
                        const rhz::ChunkPrologue* pro) {
    int algo = 0;
    const rhz_status s = check_prefill(args, true, &algo);
    if (s != RHZ_OK) return s;
    // No tokens and no final state: nothing to compute or write.
    if (args->seq_len == 0 && !args->final_state) return ok();
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (algo == RHZ_ALGO_CHUNKED) {
        const size_t need = rhz::chunked_workspace_bytes(*args);
        if (need) {
            if (!args->workspace) return fail(RHZ_ERR_WORKSPACE, "workspace is NULL (%zu bytes needed)", need);
            if (args->workspace_bytes < need)
                return fail(RHZ_ERR_WORKSPACE, "workspace has %zu bytes, %zu needed", args->workspace_bytes, need);
            if (reinterpret_cast<uintptr_t>(args->workspace) & 255u)
                return fail(RHZ_ERR_WORKSPACE, "workspace must be 256-byte aligned");
        }
        return hip_status(rhz::launch_chunked(*args, st, spin_limit, pro), "chunked prefill launch");
    }
    return hip_status(rhz::launch_recurrent(*args, st), "recurrent prefill launch");
}
}  // namespace

extern "C" {

rhz_status rhz_gdr_decode_step(const rhz_gdr_decode_args* a, void* stream) {
    if (!a) return fail(RHZ_ERR_INVALID_ARG, "args is NULL");
    if (a->batch < 1) return fail(RHZ_ERR_INVALID_ARG, "batch must be >= 1 (got %d)", a->batch);
    if (a->heads < 1) return fail(RHZ_ERR_INVALID_ARG, "heads must be >= 1 (got %d)", a->heads);
    if (a->d_k < 1) return fail(RHZ_ERR_INVALID_ARG, "d_k must be >= 1 (got %d)", a->d_k);
    if (a->d_v < 1) return fail(RHZ_ERR_INVALID_ARG, "d_v must be >= 1 (got %d)", a->d_v);
    if (a->dtype != RHZ_F32 && a->dtype != RHZ_BF16)
        return fail(RHZ_ERR_INVALID_ARG, "dtype must be RHZ_F32 or RHZ_BF16 (got %d)", a->dtype);
    if (a->gate_kind != RHZ_GATE_LOG_ALPHA && a->gate_kind != RHZ_GATE_ALPHA)
        return fail(RHZ_ERR_INVALID_ARG, "gate_kind must be RHZ_GATE_LOG_ALPHA or RHZ_GATE_ALPHA (got %d)",
                    a->gate_kind);
    if (a->d_k > 256) return fail(RHZ_ERR_UNSUPPORTED, "d_k = %d exceeds the supported 256", a->d_k);
    if (a->d_v > 1024) return fail(RHZ_ERR_UNSUPPORTED, "d_v = %d exceeds the supported 1024", a->d_v);
    if ((int64_t)a->batch * a->heads > kMaxIndex) return fail(RHZ_ERR_INVALID_ARG, "batch * heads exceeds 2^31 - 1");
    if (!a->q) return fail(RHZ_ERR_INVALID_ARG, "q is NULL");
    if (!a->k) return fail(RHZ_ERR_INVALID_ARG, "k is NULL");
    if (!a->v) return fail(RHZ_ERR_INVALID_ARG, "v is NULL");
    if (!a->gate) return fail(RHZ_ERR_INVALID_ARG, "gate is NULL");
    if (!a->beta) return fail(RHZ_ERR_INVALID_ARG, "beta is NULL");
    if (!a->state) return fail(RHZ_ERR_INVALID_ARG, "state is NULL");
    if (!a->o) return fail(RHZ_ERR_INVALID_ARG, "o is NULL");
    const size_t ea = a->dtype == RHZ_F32 ? 4 : 2;
    const void* ptrs[] = {a->q, a->k, a->v, a->o};
    const char* names[] = {"q", "k", "v", "o"};
    for (int i = 0; i < 4; ++i)
        if (reinterpret_cast<uintptr_t>(ptrs[i]) % ea)
            return fail(RHZ_ERR_INVALID_ARG, "%s is not aligned to its element size", names[i]);
    if (reinterpret_cast<uintptr_t>(a->gate) % 4 || reinterpret_cast<uintptr_t>(a->beta) % 4 ||
        reinterpret_cast<uintptr_t>(a->state) % 4)
        return fail(RHZ_ERR_INVALID_ARG, "fp32 tensors must be 4-byte aligned");
    return hip_status(rhz::launch_decode(*a, static_cast<hipStream_t>(stream)), "decode step launch");
}

rhz_status rhz_gdr_multistep(const rhz_gdr_multistep_args* a, void* stream) {
    if (!a) return fail(RHZ_ERR_INVALID_ARG, "args is NULL");
    if (a->batch < 1) return fail(RHZ_ERR_INVALID_ARG, "batch must be >= 1 (got %d)", a->batch);
    if (a->steps < 1) return fail(RHZ_ERR_INVALID_ARG, "steps must be >= 1 (got %d)", a->steps);
    if (a->heads < 1) return fail(RHZ_ERR_INVALID_ARG, "heads must be >= 1 (got %d)", a->heads);
    if (a->d_k < 1) return fail(RHZ_ERR_INVALID_ARG, "d_k must be >= 1 (got %d)", a->d_k);
    if (a->d_v < 1) return fail(RHZ_ERR_INVALID_ARG, "d_v must be >= 1 (got %d)", a->d_v);
    if (a->dtype != RHZ_F32 && a->dtype != RHZ_BF16)
        return fail(RHZ_ERR_INVALID_ARG, "dtype must be RHZ_F32 or RHZ_BF16 (got %d)", a->dtype);
    if (a->gate_kind != RHZ_GATE_LOG_ALPHA && a->gate_kind != RHZ_GATE_ALPHA)
        return fail(RHZ_ERR_INVALID_ARG, "gate_kind must be RHZ_GATE_LOG_ALPHA or RHZ_GATE_ALPHA (got %d)",
                    a->gate_kind);
    if (a->steps > RHZ_MULTISTEP_MAX)
        return fail(RHZ_ERR_UNSUPPORTED, "steps = %d exceeds the supported %d", a->steps, RHZ_MULTISTEP_MAX);
    if (a->d_k > 256) return fail(RHZ_ERR_UNSUPPORTED, "d_k = %d exceeds the supported 256", a->d_k);
    if (a->d_v > 1024) return fail(RHZ_ERR_UNSUPPORTED, "d_v = %d exceeds the supported 1024", a->d_v);
    if ((int64_t)a->batch * a->heads * a->steps > kMaxIndex)
        return fail(RHZ_ERR_INVALID_ARG, "batch * steps * heads exceeds 2^31 - 1");
    if (!a->q) return fail(RHZ_ERR_INVALID_ARG, "q is NULL");
    if (!a->k) return fail(RHZ_ERR_INVALID_ARG, "k is NULL");
    if (!a->v) return fail(RHZ_ERR_INVALID_ARG, "v is NULL");
    if (!a->gate) return fail(RHZ_ERR_INVALID_ARG, "gate is NULL");
    if (!a->beta) return fail(RHZ_ERR_INVALID_ARG, "beta is NULL");
    if (!a->state) return fail(RHZ_ERR_INVALID_ARG, "state is NULL");
    if (!a->states) return fail(RHZ_ERR_INVALID_ARG, "states is NULL");
    if (!a->o) return fail(RHZ_ERR_INVALID_ARG, "o is NULL");
    const size_t ea = a->dtype == RHZ_F32 ? 4 : 2;
    const void* ptrs[] = {a->q, a->k, a->v, a->o};
    const char* names[] = {"q", "k", "v", "o"};
    for (int i = 0; i < 4; ++i)
        if (reinterpret_cast<uintptr_t>(ptrs[i]) % ea)
            return fail(RHZ_ERR_INVALID_ARG, "%s is not aligned to its element size", names[i]);
    if (reinterpret_cast<uintptr_t>(a->gate) % 4 || reinterpret_cast<uintptr_t>(a->beta) % 4 ||
        reinterpret_cast<uintptr_t>(a->state) % 4 || reinterpret_cast<uintptr_t>(a->states) % 4)
        return fail(RHZ_ERR_INVALID_ARG, "fp32 tensors must be 4-byte aligned");
    return hip_status(rhz::launch_multistep(*a, static_cast<hipStream_t>(stream)), "multistep launch");
}

namespace {
bool misaligned(const void* p, size_t a) { return reinterpret_cast<uintptr_t>(p) % a != 0; }
}  // namespace

rhz_status rhz_causal_conv1d(const rhz_conv1d_args* a, void* stream) {
    if (!a) return fail(RHZ_ERR_INVALID_ARG, "args is NULL");
    if (a->batch < 1) return fail(RHZ_ERR_INVALID_ARG, "batch must be >= 1 (got %d)", a->batch);
    if (a->seq_len < 0) return fail(RHZ_ERR_INVALID_ARG, "seq_len must be >= 0 (got %d)", a->seq_len);
    if (a->channels < 1) return fail(RHZ_ERR_INVALID_ARG, "channels must be >= 1 (got %d)", a->channels);
    if (a->dtype != RHZ_F32 && a->dtype != RHZ_BF16)
        return fail(RHZ_ERR_INVALID_ARG, "dtype must be RHZ_F32 or RHZ_BF16 (got %d)", a->dtype);
    const int64_t tokens = a->cu_seqlens ? a->seq_len : (int64_t)a->batch * a->seq_len;
    if (tokens * a->channels > kMaxIndex || (int64_t)a->batch * a->channels * 3 > kMaxIndex)
        return fail(RHZ_ERR_INVALID_ARG, "tokens * channels and batch * channels * 3 must stay below 2^31");
    if (tokens > 0 && (!a->x || !a->y)) return fail(RHZ_ERR_INVALID_ARG, "x or y is NULL");
    if (!a->weight) return fail(RHZ_ERR_INVALID_ARG, "weight is NULL");
    const size_t ea = a->dtype == RHZ_F32 ? 4 : 2;
    if (misaligned(a->x, ea) || misaligned(a->y, ea))
        return fail(RHZ_ERR_INVALID_ARG, "x or y is not aligned to its element size");
    if (misaligned(a->weight, 4) || misaligned(a->bias, 4) || misaligned(a->initial_state, 4) ||
        misaligned(a->final_state, 4) || misaligned(a->cu_seqlens, 4))
        return fail(RHZ_ERR_INVALID_ARG, "fp32 and int32 tensors must be 4-byte aligned");
    return hip_status(rhz::launch_conv1d(*a, static_cast<hipStream_t>(stream)), "conv1d launch");
}

rhz_status rhz_gdr_prepare(const rhz_gdr_prepare_args* a, void* stream) {
    if (!a) return fail(RHZ_ERR_INVALID_ARG, "args is NULL");
    if (a->tokens < 0) return fail(RHZ_ERR_INVALID_ARG, "tokens must be >= 0 (got %d)", a->tokens);
    if (a->heads < 1) return fail(RHZ_ERR_INVALID_ARG, "heads must be >= 1 (got %d)", a->heads);
    if (a->d_k < 1) return fail(RHZ_ERR_INVALID_ARG, "d_k must be >= 1 (got %d)", a->d_k);
    if (a->dtype != RHZ_F32 && a->dtype != RHZ_BF16)
        return fail(RHZ_ERR_INVALID_ARG, "dtype must be RHZ_F32 or RHZ_BF16 (got %d)", a->dtype);
    if (a->d_k > 256) return fail(RHZ_ERR_UNSUPPORTED, "d_k = %d exceeds the supported 256", a->d_k);
    if ((int64_t)a->tokens * a->heads * a->d_k > kMaxIndex)
        return fail(RHZ_ERR_INVALID_ARG, "tokens * heads * d_k exceeds 2^31 - 1");
    if (!std::isfinite(a->q_scale)) return fail(RHZ_ERR_INVALID_ARG, "q_scale must be finite");
    if (a->tokens == 0) return ok();
    const void* ptrs[] = {a->q_in, a->k_in, a->q_out, a->k_out, a->beta_logit, a->alpha_logit, a->a_log,
                          a->beta, a->g};
    const char* names[] = {"q_in", "k_in", "q_out", "k_out", "beta_logit", "alpha_logit", "a_log", "beta", "g"};
    for (int i = 0; i < 9; ++i)
        if (!ptrs[i]) return fail(RHZ_ERR_INVALID_ARG, "%s is NULL", names[i]);
    const size_t ea = a->dtype == RHZ_F32 ? 4 : 2;
    for (int i = 0; i < 9; ++i)
        if (misaligned(ptrs[i], i < 4 ? ea : 4)) return fail(RHZ_ERR_INVALID_ARG, "%s is not aligned", names[i]);
    return hip_status(rhz::launch_prepare(*a, static_cast<hipStream_t>(stream)), "prepare launch");
}

rhz_status rhz_gdr_conv_prepare(const rhz_gdr_conv_prepare_args* a, void* stream) {
    if (!a) return fail(RHZ_ERR_INVALID_ARG, "args is NULL");
    if (a->batch < 1) return fail(RHZ_ERR_INVALID_ARG, "batch must be >= 1 (got %d)", a->batch);
    if (a->seq_len < 0) return fail(RHZ_ERR_INVALID_ARG, "seq_len must be >= 0 (got %d)", a->seq_len);
    if (a->heads < 1) return fail(RHZ_ERR_INVALID_ARG, "heads must be >= 1 (got %d)", a->heads);
    if (a->d_k < 1 || a->d_v < 1)
        return fail(RHZ_ERR_INVALID_ARG, "d_k and d_v must be >= 1 (got %d, %d)", a->d_k, a->d_v);
    if (a->dtype != RHZ_F32 && a->dtype != RHZ_BF16)
        return fail(RHZ_ERR_INVALID_ARG, "dtype must be RHZ_F32 or RHZ_BF16 (got %d)", a->dtype);
    if (!std::isfinite(a->q_scale)) return fail(RHZ_ERR_INVALID_ARG, "q_scale must be finite");
    if (a->d_k > 512 || a->d_v > 1024)
        return fail(RHZ_ERR_UNSUPPORTED, "d_k = %d, d_v = %d exceed the supported 512 and 1024", a->d_k, a->d_v);
    if (!rhz::conv_prepare_supported(a->dtype, a->d_k, a->d_v))
        return fail(RHZ_ERR_UNSUPPORTED,
                    "d_k = %d, d_v = %d: need multiples of %d with d_k / %d a power of two up to 64 "
                    "(use rhz_causal_conv1d and rhz_gdr_prepare)",
                    a->d_k, a->d_v, a->dtype == RHZ_F32 ? 4 : 8, a->dtype == RHZ_F32 ? 4 : 8);
    const int64_t C = (int64_t)a->heads * (2 * a->d_k + a->d_v);
    const int64_t tokens = a->cu_seqlens ? a->seq_len : (int64_t)a->batch * a->seq_len;
    if (tokens * C > kMaxIndex || (int64_t)a->batch * C * 3 > kMaxIndex)
        return fail(RHZ_ERR_INVALID_ARG, "tokens * channels and batch * channels * 3 must stay below 2^31");
    if (!a->weight) return fail(RHZ_ERR_INVALID_ARG, "weight is NULL");
    if (tokens > 0) {
        const void* ptrs[] = {a->x, a->q, a->k, a->v, a->beta_logit, a->alpha_logit, a->a_log, a->beta, a->g};
        const char* names[] = {"x", "q", "k", "v", "beta_logit", "alpha_logit", "a_log", "beta", "g"};
        for (int i = 0; i < 9; ++i)
            if (!ptrs[i]) return fail(RHZ_ERR_INVALID_ARG, "%s is NULL", names[i]);
        for (int i = 0; i < 4; ++i)
            if (!aligned16(ptrs[i])) return fail(RHZ_ERR_INVALID_ARG, "%s is not 16-byte aligned", names[i]);
        // x must not overlap an output: every token's outputs are written
        // while other blocks still read x
        const size_t es = a->dtype == RHZ_F32 ? 4 : 2;
        const uintptr_t x0 = reinterpret_cast<uintptr_t>(a->x), x1 = x0 + (size_t)(tokens * C) * es;
        const size_t nout[] = {(size_t)(tokens * a->heads * a->d_k) * es, (size_t)(tokens * a->heads * a->d_k) * es,
                               (size_t)(tokens * a->heads * a->d_v) * es};
        for (int i = 0; i < 3; ++i) {
            const uintptr_t o0 = reinterpret_cast<uintptr_t>(ptrs[1 + i]), o1 = o0 + nout[i];
            if (o0 < x1 && x0 < o1) return fail(RHZ_ERR_INVALID_ARG, "%s overlaps x", names[1 + i]);
        }
    }
    if (misaligned(a->weight, 4) || misaligned(a->bias, 4) || misaligned(a->initial_state, 4) ||
        misaligned(a->final_state, 4) || misaligned(a->cu_seqlens, 4) || misaligned(a->beta_logit, 4) ||
        misaligned(a->alpha_logit, 4) || misaligned(a->a_log, 4) || misaligned(a->beta, 4) || misaligned(a->g, 4))
        return fail(RHZ_ERR_INVALID_ARG, "fp32 and int32 tensors must be 4-byte aligned");
    return hip_status(rhz::launch_conv_prepare(*a, static_cast<hipStream_t>(stream)), "conv prepare launch");
}

rhz_status rhz_rmsnorm_heads(const rhz_rmsnorm_args* a, void* stream) {
    if (!a) return fail(RHZ_ERR_INVALID_ARG, "args is NULL");
    if (a->rows < 0) return fail(RHZ_ERR_INVALID_ARG, "rows must be >= 0 (got %d)", a->rows);
    if (a->dim < 1) return fail(RHZ_ERR_INVALID_ARG, "dim must be >= 1 (got %d)", a->dim);
    if (a->dtype != RHZ_F32 && a->dtype != RHZ_BF16)
        return fail(RHZ_ERR_INVALID_ARG, "dtype must be RHZ_F32 or RHZ_BF16 (got %d)", a->dtype);
    if (a->dim > 1024) return fail(RHZ_ERR_UNSUPPORTED, "dim = %d exceeds the supported 1024", a->dim);
    if (!(a->eps >= 0.f)) return fail(RHZ_ERR_INVALID_ARG, "eps must be >= 0");
    if ((int64_t)a->rows * a->dim > kMaxIndex) return fail(RHZ_ERR_INVALID_ARG, "rows * dim exceeds 2^31 - 1");
    if (a->rows == 0) return ok();
    if (!a->x || !a->y || !a->scale) return fail(RHZ_ERR_INVALID_ARG, "x, y or scale is NULL");
    const size_t ea = a->dtype == RHZ_F32 ? 4 : 2;
    if (misaligned(a->x, ea) || misaligned(a->y, ea) || misaligned(a->scale, 4))
        return fail(RHZ_ERR_INVALID_ARG, "x, y or scale is not aligned");
    return hip_status(rhz::launch_rmsnorm(*a, static_cast<hipStream_t>(stream)), "rmsnorm launch");
}

rhz_status rhz_philox_fill(int32_t kind, uint64_t seed, uint64_t stream_id, int64_t count, int32_t row_len,
                           double mean, double std_dev, int32_t out_dtype, void* out, void* stream) {
    if (kind < RHZ_FILL_NORMAL || kind > RHZ_FILL_UNIFORM) return fail(RHZ_ERR_INVALID_ARG, "unknown kind %d", kind);
    if (count < 0) return fail(RHZ_ERR_INVALID_ARG, "count must be >= 0");
    if (out_dtype != RHZ_F32 && out_dtype != RHZ_BF16 && out_dtype != RHZ_F64)
        return fail(RHZ_ERR_INVALID_ARG, "out_dtype must be RHZ_F64, RHZ_F32 or RHZ_BF16");
    if (kind == RHZ_FILL_UNIT_ROWS && (row_len < 1 || count % row_len != 0))
        return fail(RHZ_ERR_INVALID_ARG, "UNIT_ROWS needs row_len >= 1 dividing count");
    if (count > 0 && !out) return fail(RHZ_ERR_INVALID_ARG, "out is NULL");
    if (count > ((int64_t)1 << 40)) return fail(RHZ_ERR_INVALID_ARG, "count too large");
    return hip_status(rhz::launch_philox_fill(kind, seed, stream_id, count, row_len, mean, std_dev, out_dtype, out,
                                              static_cast<hipStream_t>(stream)),
                      "philox fill launch");
}

}  // extern "C"
