// Split-K workspace of the allocation-free attention entry point
// (dk_paged_attention_decode_noalloc, paged_attention.hip).
//
// One array per GPU, shared by every no-alloc call on that GPU (overlapping
// calls on one GPU race) and kept, with the last call's contents, until the
// process ends. Nothing in it has to start at zero: the kernels read only rows
// written by the same call.
//
// The array is the only device symbol of this source file, so it lives in a
// code object of its own. The HIP runtime loads a code object onto a device
// when one of its symbols is first used there (deferred loading, the default),
// so a process holds the array's 64 MiB on a device only after a no-alloc call
// ran on that device, not whenever the attention kernels load.
#include <atomic>

#include "../../include/decodekernels_amd.h"
#include "dk_host.h"

namespace dk {
namespace attn {

namespace {
constexpr int kMaxScratchDevices = 64;
}  // namespace

static __device__ __align__(256) unsigned char scratch[DK_NOALLOC_SCRATCH_BYTES];

// Device address of the current device's `scratch` (host code must not use the
// array's name, a host-side stand-in): looked up with hipGetSymbolAddress on
// the first call on each device, with that device current, then cached.
void* noalloc_scratch_address(int* err) {
  static std::atomic<void*> addr[kMaxScratchDevices];
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    *err = static_cast<int>(e);
    return nullptr;
  }
  if (dev < 0 || dev >= kMaxScratchDevices) {
    *err = fail("paged_attention_decode_noalloc: device %d is beyond the %d devices supported", dev,
                kMaxScratchDevices);
    return nullptr;
  }
  void* p = addr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      *err = e != hipSuccess ? static_cast<int>(e) : static_cast<int>(hipErrorInvalidSymbol);
      return nullptr;
    }
    addr[dev].store(p, std::memory_order_release);  // every thread finds the same address
  }
  return p;
}

}  // namespace attn
}  // namespace dk
