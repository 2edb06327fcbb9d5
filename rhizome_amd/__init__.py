"""rhizome_amd -- MI355X (gfx950) gated delta-rule forward behind a C ABI.

The compute lives in librhizome_gdr.so (hand-written HIP kernels, built by
``python -m rhizome_amd.build``); this package is its torch-tensor front
end.  Importing the package does not load the library; the first call does,
and raises if the library is missing.
"""
from .gdr import (causal_conv1d, conv_prepare, decode_step, exact_reruns, fp16_range_errors,  # noqa: F401
                  local_prefill, multistep, philox_fill, prefill, prepare, query_support,
                  rmsnorm_heads, sync_timeouts)

__all__ = ["prefill", "local_prefill", "decode_step", "multistep", "causal_conv1d", "prepare", "conv_prepare",
           "rmsnorm_heads", "philox_fill", "query_support", "sync_timeouts", "fp16_range_errors",
           "exact_reruns"]
