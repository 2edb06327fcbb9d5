// gdr_chunked_pre.hip -- the chunked prefill kernel's instances with the
// fused prologue (rhz_gdr_local_prefill), compiled in a unit of their own:
// the kernel source is gdr_chunked.hip, whose launch code calls
// chunked_go_prologue and chunked_prologue_counter defined here.
#define RHZ_CHUNKED_PROLOGUE_TU 1
#include "gdr_chunked.hip"
