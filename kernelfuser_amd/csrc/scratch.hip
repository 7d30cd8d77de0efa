// Static device workspace of the allocation-free attention entry point
// (kfmi_launch_attention_bf16_noalloc).  The only scratch buffer of the
// attention path is the split-KV workspace (arrival counters + FP32 partial
// results of the causal D = 256 launches that split their longest query
// blocks, see attention_workspace_bytes).  Callers that cannot allocate
// (code under HIP graph capture, tight serving loops, harnesses that forbid
// hipMalloc) get it from this file-scope array instead: each GPU the library
// runs on holds one copy of KFMI_SCRATCH_BYTES until the process ends.
//
// The array's name is a host-side stand-in: host code uses only the device
// address that hipGetSymbolAddress returns for the current device, cached per
// device ordinal.  Every call on a GPU shares that GPU's array and finds the
// last call's contents, so each call clears the counters it needs (a fill
// kernel on the caller's stream, ahead of the attention launch); calls that
// overlap in time on one GPU (two streams, or two replays of graphs that hold
// this entry point) race on it.
#include <hip/hip_runtime.h>

#include <mutex>

#include "kfmi_launch.h"

namespace kfmi {
namespace {

static __device__ __align__(256) unsigned char scratch[KFMI_SCRATCH_BYTES];

// Fill n 32-bit words with zeros (one workgroup; n is a few hundred).  A
// kernel rather than hipMemsetAsync, so that a capturing caller records an
// ordinary kernel node.
__global__ __launch_bounds__(256) void zero_words_kernel(uint32_t *p, int n) {
  for (int i = threadIdx.x; i < n; i += 256) p[i] = 0u;
}

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void *g_addr[kMaxDevices];  // device address of `scratch` per device ordinal (nullptr: not taken yet)

}  // namespace

hipError_t noalloc_scratch(void **addr) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_mu);
  if (g_addr[dev] == nullptr) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (p == nullptr) return hipErrorInvalidSymbol;
    g_addr[dev] = p;
  }
  *addr = g_addr[dev];
  return hipSuccess;
}

hipError_t clear_scratch_words(void *addr, int64_t bytes, hipStream_t stream) {
  const int n = (int)(bytes / 4);
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(zero_words_kernel, dim3(1), dim3(256), 0, stream, (uint32_t *)addr, n);
  launch_log_add(reinterpret_cast<const void *>(&zero_words_kernel), "zero_words_kernel", 1, 256);
  return hipGetLastError();
}

}  // namespace kfmi
