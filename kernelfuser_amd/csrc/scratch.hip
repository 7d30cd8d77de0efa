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

// Clock stamps of the attention launches that record them: {t0, t1, r0, r1}
// per workgroup (kfmi_clock_stamp), one array per GPU, written only by the
// launches that pass its address.
static __device__ __align__(256) unsigned long long clock_stamps[4 * KFMI_CLOCK_STAMPS_MAX];

// Fill n 32-bit words with zeros (one workgroup; n is a few hundred).  A
// kernel rather than hipMemsetAsync, so that a capturing caller records an
// ordinary kernel node.
__global__ __launch_bounds__(256) void zero_words_kernel(uint32_t *p, int n) {
  for (int i = threadIdx.x; i < n; i += 256) p[i] = 0u;
}

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void *g_addr[kMaxDevices];  // device address of `scratch` per device ordinal (nullptr: not taken yet)
void *g_stamp_addr[kMaxDevices];  // device address of `clock_stamps` per device ordinal
int g_stamp_count[kMaxDevices];   // entries written by the last recording launch per device

// Address of `sym` on the current device, cached in cache[device].
hipError_t symbol_address(const void *sym, void **cache, void **addr) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_mu);
  if (cache[dev] == nullptr) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, sym);
    if (e != hipSuccess) return e;
    if (p == nullptr) return hipErrorInvalidSymbol;
    cache[dev] = p;
  }
  *addr = cache[dev];
  return hipSuccess;
}

}  // namespace

hipError_t noalloc_scratch(void **addr) { return symbol_address(HIP_SYMBOL(scratch), g_addr, addr); }

hipError_t clock_stamp_buffer(void **addr) { return symbol_address(HIP_SYMBOL(clock_stamps), g_stamp_addr, addr); }

void clock_stamps_recorded(int64_t workgroups) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return;
  std::lock_guard<std::mutex> lock(g_mu);
  g_stamp_count[dev] = (int)(workgroups < KFMI_CLOCK_STAMPS_MAX ? workgroups : KFMI_CLOCK_STAMPS_MAX);
}

int clock_stamps_count() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 0;
  std::lock_guard<std::mutex> lock(g_mu);
  return g_stamp_count[dev];
}

hipError_t clear_scratch_words(void *addr, int64_t bytes, hipStream_t stream) {
  const int n = (int)(bytes / 4);
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(zero_words_kernel, dim3(1), dim3(256), 0, stream, (uint32_t *)addr, n);
  launch_log_add(reinterpret_cast<const void *>(&zero_words_kernel), "zero_words_kernel", 1, 256);
  return hipGetLastError();
}

}  // namespace kfmi
