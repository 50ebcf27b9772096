// The fixed scratch of ltx25_linear_q_noalloc: the split-K f32 partials
// live in a file-scope device array instead of the library's grow-only
// heap buffer, so that entry point never allocates. It is for callers that
// cannot call hipMalloc: code under HIP graph capture, tight serving loops,
// harnesses that forbid allocation.
//
// Every GPU the library runs on holds its own copy of the array, at its
// own address, until the process ends. Host code never passes the array's
// name to a kernel or a copy: on the host that name is only a stand-in, and
// a kernel handed it would fault. noalloc_scratch() resolves the device's
// real address once per device (hipGetSymbolAddress with that device
// current) and every use goes through that pointer.
#include "common.h"

#include <hip/hip_runtime.h>

#include <mutex>

namespace {

constexpr int kScratchDevices = 64;

// Split-K partials of one call: splits x M x N floats. Every plan the
// planner makes for a 256-CU device fits: the M <= 128 kernel keeps
// (N / 32) x splits within three workgroups per CU and the 128 x 128 tile
// splits only until its workgroups cover the CUs once (the largest found
// is 31.6 MiB: 127 rows x 32640 columns x 2 splits).
static __device__ __align__(256) unsigned char scratch[ltx25::kNoAllocScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[kScratchDevices] = {};

}  // namespace

namespace ltx25 {

hipError_t noalloc_scratch(void** out)
{
  *out = nullptr;
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) { return e; }
  if (dev < 0 || dev >= kScratchDevices) { return hipErrorInvalidDevice; }
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) { return e; }
    if (p == nullptr) { return hipErrorInvalidSymbol; }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return hipSuccess;
}

}  // namespace ltx25
