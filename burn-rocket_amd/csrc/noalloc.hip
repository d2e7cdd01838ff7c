// Static device scratch of the entry point that allocates nothing
// (rk_attention_dev_noalloc): the Vᵀ operand of the attention kernel lives in
// a file-scope device array instead of hipMalloc'd library scratch, for
// callers that cannot allocate (graph capture, serving loops).
#include "common.hpp"
#include "kernels.hpp"

// RK_NOALLOC_SCRATCH_BYTES (32 MiB): Vᵀ of up to 8 kv heads × 128 values ×
// 16384 keys in fp16. Each GPU the library runs on holds its own copy until
// the process ends. Host code must not use the array's name as an address:
// kernels get the per-device pointer that rk_noalloc_setup looks up.
static __device__ __align__(256) uint8_t scratch[RK_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
void *g_scratch_ptr[kMaxDevices];  // this file's `scratch` on each device (null: not set up)
}  // namespace

hipError_t rk_noalloc_setup(int device) {
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  if (g_scratch_ptr[device]) return hipSuccess;
  void *p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess) return e;
  if (!p) return hipErrorInvalidSymbol;
  g_scratch_ptr[device] = p;
  return hipSuccess;
}

void *rk_noalloc_scratch(int device) {
  return (device >= 0 && device < kMaxDevices) ? g_scratch_ptr[device] : nullptr;
}
