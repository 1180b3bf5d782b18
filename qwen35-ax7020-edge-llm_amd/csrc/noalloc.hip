// noalloc.hip -- the device scratch of bfp8_dev_lm_head_topk_noalloc, the
// variant of bfp8_dev_lm_head_topk for callers that cannot allocate device
// memory (code under HIP graph capture, tight serving loops, harnesses that
// forbid hipMalloc).
//
// The scratch is one file-scope device array of a fixed size; every GPU the
// library runs on holds its own copy until the process ends.  In host code the
// array's name is only a stand-in: its device address is looked up once per
// device with hipGetSymbolAddress and only that address is ever passed on.
#include <hip/hip_runtime.h>

#include "bfp8_internal.h"

// Partial top-k lists (BFP8_NOALLOC_MAX_VOCAB / 64 tiles x BFP8_TOPK_MAX keys),
// the scores of every row, the sort keys of every row.
constexpr size_t kScratchBytes = BFP8_NOALLOC_PARTIALS_BYTES + BFP8_NOALLOC_LOGITS_BYTES + BFP8_NOALLOC_KEYS_BYTES;
static __device__ __align__(256) uint64_t scratch[kScratchBytes / 8];

namespace {
constexpr int kMaxDevices = 64;
void* g_scratch_ptr[kMaxDevices];  // device address of `scratch`, per device (null: not looked up yet)
}  // namespace

hipError_t bfp8_noalloc_setup(void** out) {
    *out = nullptr;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return hipSuccess;
}
