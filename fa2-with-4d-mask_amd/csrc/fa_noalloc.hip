// Device scratch of the allocation-free backward entry point (fa_bwd_noalloc).
//
// The backward needs, beyond its inputs and outputs, Delta and the backward's
// LSE (2 floats per query row of every head) and one dead-row flag per
// (batch, kv-head).  fa_bwd takes them as caller workspaces; fa_bwd_noalloc
// keeps them in this file-scope array instead, so that callers that cannot
// allocate device memory (code under HIP graph capture, serving loops,
// harnesses that forbid hipMalloc) can run the backward.  Each GPU the
// library runs on holds its own copy of the array until the process ends.
//
// Host code never uses the array's name as an address (in host code it is a
// stand-in, not the device location): scratch_device_ptr() looks the device
// address up with hipGetSymbolAddress once per device, with that device
// current, and every kernel argument uses that address.
//
// Every call on one GPU shares the array and it keeps the previous call's
// contents: the flags are cleared by a fill kernel at the start of every
// call (a kernel, not hipMemsetAsync, so the call can be captured into a
// graph), and calls that overlap on one GPU (different streams, or host
// threads without ordering) race on it.
#include <hip/hip_runtime.h>

#include <mutex>

#include "fa_kernels.h"

namespace fa {

constexpr int64_t kNoallocScratchBytes = 16ll << 20;   // 16 MiB per GPU
constexpr int kMaxDevices = 64;

static __device__ __align__(256) char scratch[kNoallocScratchBytes];

namespace {

std::mutex g_mu;
void* g_ptr[kMaxDevices] = {};

__global__ void fill_i32_kernel(int32_t* p, int64_t n, int32_t v) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = v;
}

}  // namespace

int64_t noalloc_scratch_bytes() { return kNoallocScratchBytes; }

// Device address of this GPU's scratch array (the current device's), looked
// up once per device; hipSuccess or the lookup's error.
hipError_t scratch_device_ptr(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    g_ptr[dev] = p;
  }
  *out = g_ptr[dev];
  return hipSuccess;
}

hipError_t launch_fill_i32(int32_t* p, int64_t n, int32_t v, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  int64_t blocks = (n + 255) / 256;
  if (blocks > 1024) blocks = 1024;
  hipLaunchKernelGGL(fill_i32_kernel, dim3((unsigned)blocks), dim3(256), 0, s, p, n, v);
  return hipGetLastError();
}

}  // namespace fa
