// Host-side launch descriptors shared by the C ABI and the kernel files.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kfmi.h"

namespace kfmi {

// Row styles of the preparation and attention-prologue arithmetic.
enum Style : int {
  ST_HF = 0,       // BF16 at each HF op boundary (norm, x gamma, each RoPE product, +/-)
  ST_LEGACY = 1,   // one BF16 cast of x*inv*gamma, then the BF16 RoPE chain
  ST_FP32 = 2,     // FP32 throughout, one final BF16 rounding
  ST_FACTORED = 3  // Q rows -> FP32 inverse RMS; K rows -> bf16(k*inv*gk*gq)
};

// Attention prologue kinds.
enum Prologue : int {
  PRO_NONE = 0,          // Q already prepared
  PRO_NORM = 1,          // Q RMSNorm in the prologue
  PRO_NORM_ROPE = 2,     // Q RMSNorm + rotate-half RoPE in the prologue
  PRO_FACTORED_READ = 3, // raw Q, per-row inverse RMS read from inv[]
  PRO_FACTORED_CALC = 4  // raw Q, per-row inverse RMS computed (and written to inv[])
};

struct RowsArgs {
  const uint16_t *q, *k, *gq, *gk, *cos, *sin;
  uint16_t *qn, *kn;
  float *inv;
  const uint16_t *v;  // with vt: V to transpose per head in the same launch (D = 128, S % 8 == 0)
  uint16_t *vt;       // NULL: no transpose
  int64_t B, Hq, Hkv, S, D;
  bool only_k, rope;
  int style;
  float eps;
};

struct AttnArgs {
  const uint16_t *q, *k, *v, *gq, *cos, *sin;
  const uint16_t *gk;  // mode 'full': K is raw and normalised (+RoPE) per tile with this gamma; else NULL
  const uint16_t *vt;  // V transposed per head ([B,Hkv,D,S]) or NULL
  uint16_t *out;
  float *inv;
  int64_t B, Hq, Hkv, S, D;
  bool causal;
  int prologue, style;
  double scale;  // multiplies q.k (ignored by the factored prologues: D^-1/2)
  float eps;
  int bm, bn;
  void *work;          // split-KV workspace (counters + partial results) or NULL
  int64_t work_bytes;  // its size; too small = no split
};

// Both return hipSuccess or the launch error.  Arguments are validated by the caller.
// Launch log of the calling thread: each C-ABI compute entry point clears it
// once its arguments are valid, and every kernel launch appends the kernel
// instance, its grid and block and the runtime's resource figures for it.
void launch_log_clear();
void launch_log_add(const void *fn, const char *name, int64_t grid, int block);
// printf-style plan string of the last logged launch (kfmi_launch_info.plan)
void launch_log_plan(const char *fmt, ...);
inline const char *tf(bool b) { return b ? "true" : "false"; }

hipError_t launch_rows(const RowsArgs &a, hipStream_t stream);
// vt[b,h,d,s] = v[b,h,s,d] for the B*H heads of S rows of D.
hipError_t launch_transpose_v(const uint16_t *v, uint16_t *vt, int64_t BH, int64_t S, int64_t D, hipStream_t stream);
hipError_t launch_attention(const AttnArgs &a, hipStream_t stream);
// The calling thread's dispatch overrides (kfmi_set_tuning; all zero unless set).
const kfmi_tuning &thread_tuning();
// The attention kernel (KFMI_KERNEL_GENERAL / _PINGPONG / _WIDE) that
// launch_attention runs for this shape under the thread's overrides; `full`
// is mode 'full' (always the general kernel).
int attention_kernel(int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t D, bool causal, bool full);
// Why the thread's overrides cannot run this geometry (NULL: they can).
const char *attention_tuning_error(int64_t Hq, int64_t Hkv, int64_t D, bool full);
// Workspace bytes with which launch_attention splits the key range of the
// longest causal query blocks over two workgroups (0: this shape never splits).
int64_t attention_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t D, bool causal);
// Leading bytes of that workspace that hold the arrival counters, which must
// be zero when a launch starts (0: this shape never splits).
int64_t attention_workspace_counter_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t D, bool causal);

// Static split-KV workspace of the allocation-free entry point (one per GPU):
// 36 MiB covers every causal D = 256 split plan of up to 141 (block, head)
// pairs (4 KiB of counters, 260 KiB of partials per pair), which includes
// the Gemma-3 geometries up to their largest one-workgroup-per-CU grids (at
// most 128 pairs, 32.5 MiB).
#define KFMI_SCRATCH_BYTES (36ll << 20)
// Device address of the current device's static workspace (taken once per
// device with hipGetSymbolAddress and cached).
hipError_t noalloc_scratch(void **addr);
// Zero the first `bytes` (a multiple of 4) of the static workspace on `stream`
// with a fill kernel.
hipError_t clear_scratch_words(void *addr, int64_t bytes, hipStream_t stream);

// Device address of the current device's static clock-stamp array
// (4 * KFMI_CLOCK_STAMPS_MAX 64-bit words; taken once per device with
// hipGetSymbolAddress and cached), and the number of entries the last
// recording launch on each device wrote.
hipError_t clock_stamp_buffer(void **addr);
void clock_stamps_recorded(int64_t workgroups);
int clock_stamps_count();

}  // namespace kfmi
