// C ABI of the gfx950 attention-prologue library (declared in include/kfmi.h).
// Validates every argument before enqueuing anything, then dispatches to the
// kernel launchers.  No allocation, no synchronisation.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

#include "kfmi.h"
#include "kfmi_launch.h"

#include <unordered_map>
#include <vector>

namespace {

thread_local std::string g_error;
thread_local std::vector<kfmi_launch_info> g_launches;
thread_local kfmi_tuning g_tuning{};

int fail(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
  g_launches.clear();  // a failed call reports no launches
  return code;
}

int launch_status(hipError_t e, const char *what) {
  if (e != hipSuccess) return fail(KFMI_ELAUNCH, "%s: %s", what, hipGetErrorString(e));
  g_error.clear();
  return KFMI_OK;
}

}  // namespace

namespace kfmi {

const kfmi_tuning &thread_tuning() { return g_tuning; }

void launch_log_clear() { g_launches.clear(); }

void launch_log_add(const void *fn, const char *name, int64_t grid, int block) {
  // hipFuncGetAttributes once per kernel instance (the figures do not change)
  static std::mutex mu;
  static std::unordered_map<const void *, hipFuncAttributes> cache;
  hipFuncAttributes attr{};
  {
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find(fn);
    if (it == cache.end()) {
      if (hipFuncGetAttributes(&attr, fn) != hipSuccess) {
        (void)hipGetLastError();  // a failed query must not look like a failed launch
        attr = hipFuncAttributes{};
      }
      it = cache.emplace(fn, attr).first;
    }
    attr = it->second;
  }
  kfmi_launch_info r{};
  snprintf(r.kernel, sizeof(r.kernel), "%s", name);
  r.grid = grid;
  r.block = block;
  r.registers = attr.numRegs;
  r.lds_bytes = (int32_t)attr.sharedSizeBytes;
  r.scratch_bytes = (int32_t)attr.localSizeBytes;
  g_launches.push_back(r);
}

void launch_log_plan(const char *fmt, ...) {
  if (g_launches.empty()) return;
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_launches.back().plan, sizeof(g_launches.back().plan), fmt, ap);
  va_end(ap);
}

}  // namespace kfmi

namespace {

// gfx950 check of the current device, cached per device ordinal.  Every
// compute entry point calls it after its argument checks, right before it
// launches, so this is also where the call's launch log starts.
int check_device() {
  kfmi::launch_log_clear();
  static std::mutex mu;
  static int cached[64];  // 0 unknown, 1 ok, 2 wrong arch
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(KFMI_EDEVICE, "hipGetDevice failed");
  if (dev < 0 || dev >= 64) return fail(KFMI_EDEVICE, "device ordinal %d out of range", dev);
  std::lock_guard<std::mutex> lock(mu);
  if (cached[dev] == 0) {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return fail(KFMI_EDEVICE, "hipGetDeviceProperties failed");
    cached[dev] = strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 2;
    if (cached[dev] == 2) return fail(KFMI_EDEVICE, "device %d is %s; this library is built for gfx950", dev, prop.gcnArchName);
  }
  if (cached[dev] == 2) return fail(KFMI_EDEVICE, "device %d is not gfx950", dev);
  return KFMI_OK;
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Shape rules shared by all entry points (rope:705-717).
int check_shape(int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t D) {
  if (B < 1 || Hq < 1 || Hkv < 1 || S < 1) return fail(KFMI_EINVAL, "B, Hq, Hkv and S must be >= 1 (got %lld, %lld, %lld, %lld)",
                                                      (long long)B, (long long)Hq, (long long)Hkv, (long long)S);
  if (D != 128 && D != 256) return fail(KFMI_EINVAL, "D must be 128 or 256 (got %lld)", (long long)D);
  if (Hq % Hkv != 0) return fail(KFMI_EINVAL, "Hq (%lld) must be a multiple of Hkv (%lld)", (long long)Hq, (long long)Hkv);
  const int64_t lim = (int64_t)1 << 31;
  if (B * Hq * S * D >= lim || B * Hkv * S * D >= lim) return fail(KFMI_EINVAL, "tensors must have fewer than 2^31 elements");
  return KFMI_OK;
}

int check_ptrs(std::initializer_list<std::pair<const void *, const char *>> ptrs) {
  for (auto &pr : ptrs) {
    if (pr.first == nullptr) return fail(KFMI_EINVAL, "%s must not be NULL", pr.second);
    if (!aligned16(pr.first)) return fail(KFMI_EINVAL, "%s must be 16-byte aligned", pr.second);
  }
  return KFMI_OK;
}

int check_style(int norm_style) {
  if (norm_style != KFMI_NORM_HF && norm_style != KFMI_NORM_LEGACY && norm_style != KFMI_NORM_FP32)
    return fail(KFMI_EINVAL, "norm_style must be KFMI_NORM_HF, KFMI_NORM_LEGACY or KFMI_NORM_FP32 (got %d)", norm_style);
  return KFMI_OK;
}

int check_tiles(int bm, int bn) {
  if (bm < 32 || bm > 256 || bm % 32 != 0) return fail(KFMI_EINVAL, "bm must be a multiple of 32 in [32, 256] (got %d)", bm);
  if (bn != 32 && bn != 64 && bn != 128) return fail(KFMI_EINVAL, "bn must be 32, 64 or 128 (got %d)", bn);
  return KFMI_OK;
}

int style_of(int norm_style) {
  return norm_style == KFMI_NORM_HF ? kfmi::ST_HF : norm_style == KFMI_NORM_LEGACY ? kfmi::ST_LEGACY : kfmi::ST_FP32;
}

#define KFMI_TRY(x)            \
  do {                         \
    int rc_ = (x);             \
    if (rc_ != KFMI_OK) return rc_; \
  } while (0)

}  // namespace

extern "C" {

int kfmi_abi_version(void) { return KFMI_ABI_VERSION; }

const char *kfmi_last_error(void) { return g_error.c_str(); }

int kfmi_set_tuning(const kfmi_tuning *t) {
  if (t == nullptr) {
    g_tuning = kfmi_tuning{};
    g_error.clear();
    return KFMI_OK;
  }
  if (t->attn_kernel < KFMI_KERNEL_AUTO || t->attn_kernel > KFMI_KERNEL_WIDE)
    return fail(KFMI_EINVAL, "attn_kernel must be KFMI_KERNEL_AUTO .. KFMI_KERNEL_WIDE (got %d)", t->attn_kernel);
  if (t->pp_heads < 0 || t->pp_heads > 2) return fail(KFMI_EINVAL, "pp_heads must be 0, 1 or 2 (got %d)", t->pp_heads);
  if (t->rows_heads != 0 && t->rows_heads != 2 && t->rows_heads != 4)
    return fail(KFMI_EINVAL, "rows_heads must be 0, 2 or 4 (got %d)", t->rows_heads);
  if (t->split < 0 || t->split > 1) return fail(KFMI_EINVAL, "split must be 0 or 1 (got %d)", t->split);
  if (t->persistent < 0 || t->persistent > 1) return fail(KFMI_EINVAL, "persistent must be 0 or 1 (got %d)", t->persistent);
  if (t->clock_stamps < 0 || t->clock_stamps > 1)
    return fail(KFMI_EINVAL, "clock_stamps must be 0 or 1 (got %d)", t->clock_stamps);
  g_tuning = *t;
  g_error.clear();
  return KFMI_OK;
}

void kfmi_get_tuning(kfmi_tuning *out) {
  if (out) *out = g_tuning;
}

int kfmi_clock_stamps(kfmi_clock_stamp *out, int max) {
  if (max < 0 || (max > 0 && out == nullptr)) return -fail(KFMI_EINVAL, "kfmi_clock_stamps: out is NULL or max < 0");
  if (const int rc = check_device()) return -rc;
  const int n = kfmi::clock_stamps_count();
  const int m = n < max ? n : max;
  if (m > 0) {
    void *src = nullptr;
    hipError_t e = kfmi::clock_stamp_buffer(&src);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e == hipSuccess) e = hipMemcpy(out, src, (size_t)m * sizeof(kfmi_clock_stamp), hipMemcpyDeviceToHost);
    if (e != hipSuccess) return -fail(KFMI_ELAUNCH, "kfmi_clock_stamps: %s", hipGetErrorString(e));
  }
  g_error.clear();
  return n;
}

int kfmi_last_launches(kfmi_launch_info *out, int max) {
  const int n = (int)g_launches.size();
  for (int i = 0; i < n && i < max && out; ++i) out[i] = g_launches[i];
  return n;
}

int kfmi_prepare_bf16(const void *q, const void *k, const void *v, const void *gq, const void *gk, const void *cos,
                      const void *sin, void *qn, void *kn, void *vt, int64_t B, int64_t Hq, int64_t Hkv, int64_t S,
                      int64_t D, float eps, int norm_style, int flags, void *stream) {
  KFMI_TRY(check_shape(B, Hq, Hkv, S, D));
  KFMI_TRY(check_style(norm_style));
  if (flags & ~(KFMI_PREP_ONLY_K | KFMI_PREP_ROPE)) return fail(KFMI_EINVAL, "unknown flags 0x%x", flags);
  const bool only_k = flags & KFMI_PREP_ONLY_K, rope = flags & KFMI_PREP_ROPE;
  KFMI_TRY(check_ptrs({{k, "k"}, {gk, "gk"}, {kn, "kn"}}));
  if (!only_k) KFMI_TRY(check_ptrs({{q, "q"}, {gq, "gq"}, {qn, "qn"}}));
  if (rope) KFMI_TRY(check_ptrs({{cos, "cos"}, {sin, "sin"}}));
  if (!(eps >= 0.0f)) return fail(KFMI_EINVAL, "eps must be >= 0");
  if (vt) {
    KFMI_TRY(check_ptrs({{v, "v"}, {vt, "vt"}}));
    if (D != 128 || S % 8 != 0) return fail(KFMI_EINVAL, "vt needs D == 128 and S % 8 == 0");
  }
  KFMI_TRY(check_device());
  kfmi::RowsArgs a{};
  a.v = (const uint16_t *)v; a.vt = (uint16_t *)vt;
  a.q = (const uint16_t *)q; a.k = (const uint16_t *)k; a.gq = (const uint16_t *)gq; a.gk = (const uint16_t *)gk;
  a.cos = (const uint16_t *)cos; a.sin = (const uint16_t *)sin;
  a.qn = (uint16_t *)qn; a.kn = (uint16_t *)kn; a.inv = nullptr;
  a.B = B; a.Hq = Hq; a.Hkv = Hkv; a.S = S; a.D = D;
  a.only_k = only_k; a.rope = rope; a.style = style_of(norm_style); a.eps = eps;
  return launch_status(kfmi::launch_rows(a, (hipStream_t)stream), "prepare launch");
}

// The thread's dispatch overrides must be able to run this shape.
static int check_tuning(int64_t Hq, int64_t Hkv, int64_t D, bool full) {
  const char *why = kfmi::attention_tuning_error(Hq, Hkv, D, full);
  return why ? fail(KFMI_EINVAL, "kfmi_set_tuning: %s", why) : KFMI_OK;
}

static int attention_impl(const void *q, const void *k, const void *v, const void *vt, const void *gq,
                          const void *gk, const void *cos, const void *sin, void *out, float *inv, int64_t B, int64_t Hq,
                          int64_t Hkv, int64_t S, int64_t D, double scale, float eps, int causal, int prologue,
                          int style, int bm, int bn, hipStream_t stream, void *work = nullptr,
                          int64_t work_bytes = 0) {
  kfmi::AttnArgs a{};
  a.q = (const uint16_t *)q; a.k = (const uint16_t *)k; a.v = (const uint16_t *)v; a.gq = (const uint16_t *)gq;
  a.vt = (const uint16_t *)vt;
  a.gk = (const uint16_t *)gk;
  a.cos = (const uint16_t *)cos; a.sin = (const uint16_t *)sin; a.out = (uint16_t *)out; a.inv = inv;
  a.B = B; a.Hq = Hq; a.Hkv = Hkv; a.S = S; a.D = D;
  a.causal = causal != 0; a.prologue = prologue; a.style = style; a.scale = scale; a.eps = eps;
  a.bm = bm; a.bn = bn;
  a.work = work; a.work_bytes = work_bytes;
  return launch_status(kfmi::launch_attention(a, stream), "attention launch");
}

int64_t kfmi_attention_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t D, int causal) {
  if (check_shape(B, Hq, Hkv, S, D) != KFMI_OK) return -1;
  g_error.clear();
  return kfmi::attention_workspace_bytes(B, Hq, Hkv, S, D, causal != 0);
}

int kfmi_attention_kernel(int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t D, int causal, int mode) {
  if (check_shape(B, Hq, Hkv, S, D) != KFMI_OK) return -KFMI_EINVAL;
  if (mode != KFMI_MODE_QUERY && mode != KFMI_MODE_FULL && mode != KFMI_MODE_UNFUSED) {
    fail(KFMI_EINVAL, "mode must be KFMI_MODE_QUERY, _FULL or _UNFUSED (got %d)", mode);
    return -KFMI_EINVAL;
  }
  if (check_tuning(Hq, Hkv, D, mode == KFMI_MODE_FULL) != KFMI_OK) return -KFMI_EINVAL;
  g_error.clear();
  return kfmi::attention_kernel(B, Hq, Hkv, S, D, causal != 0, mode == KFMI_MODE_FULL);
}

static int check_work(const void *work, int64_t work_bytes) {
  if (work_bytes < 0) return fail(KFMI_EINVAL, "work_bytes must be >= 0");
  if (work && !aligned16(work)) return fail(KFMI_EINVAL, "work must be 16-byte aligned");
  return KFMI_OK;
}

int kfmi_attention_bf16(const void *q, const void *k, const void *v, const void *vt, const void *gq, const void *cos,
                        const void *sin, void *out, int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t D,
                        double scale, float eps, int causal, int fuse_q, int norm_style, int bm, int bn,
                        void *work, int64_t work_bytes, void *stream) {
  KFMI_TRY(check_shape(B, Hq, Hkv, S, D));
  KFMI_TRY(check_style(norm_style));
  KFMI_TRY(check_tiles(bm, bn));
  KFMI_TRY(check_ptrs({{q, "q"}, {k, "k"}, {v, "v"}, {out, "out"}}));
  if ((cos == nullptr) != (sin == nullptr)) return fail(KFMI_EINVAL, "provide both rotary tables or neither");
  if (fuse_q) KFMI_TRY(check_ptrs({{gq, "gq"}}));
  if (fuse_q && cos) KFMI_TRY(check_ptrs({{cos, "cos"}, {sin, "sin"}}));
  if (!(scale > 0.0)) return fail(KFMI_EINVAL, "scale must be > 0");
  KFMI_TRY(check_work(work, work_bytes));
  KFMI_TRY(check_tuning(Hq, Hkv, D, false));
  KFMI_TRY(check_device());
  const int pro = !fuse_q ? kfmi::PRO_NONE : (cos ? kfmi::PRO_NORM_ROPE : kfmi::PRO_NORM);
  if (vt) KFMI_TRY(check_ptrs({{vt, "vt"}}));
  return attention_impl(q, k, v, vt, gq, nullptr, cos, sin, out, nullptr, B, Hq, Hkv, S, D, scale, eps, causal, pro,
                        style_of(norm_style), bm, bn, (hipStream_t)stream, work, work_bytes);
}

// Shared body of kfmi_launch_attention_bf16 and its allocation-free variant
// (noalloc: the split-KV workspace is the static per-GPU scratch array
// instead of the caller's `work`).
static int launch_attention_entry(const void *q, const void *k, const void *v, const void *gq, const void *gk,
                                  const void *cos, const void *sin, void *out, void *qn, void *kn, void *vt,
                                  int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t D, double scale, float eps,
                                  int causal, int mode, int norm_style, int bm, int bn, void *work,
                                  int64_t work_bytes, void *stream, bool noalloc) {
  KFMI_TRY(check_shape(B, Hq, Hkv, S, D));
  KFMI_TRY(check_style(norm_style));
  KFMI_TRY(check_tiles(bm, bn));
  if (mode != KFMI_MODE_QUERY && mode != KFMI_MODE_UNFUSED && mode != KFMI_MODE_FULL)
    return fail(KFMI_EINVAL, "Invalid fusion mode %d", mode);
  KFMI_TRY(check_ptrs({{q, "q"}, {k, "k"}, {v, "v"}, {gq, "gq"}, {gk, "gk"}, {out, "out"}}));
  KFMI_TRY(check_work(work, work_bytes));
  if (mode != KFMI_MODE_FULL) {
    if (kn == nullptr || (mode == KFMI_MODE_UNFUSED && qn == nullptr)) return fail(KFMI_EINVAL, "Missing scratch buffers");
    KFMI_TRY(check_ptrs({{kn, "kn"}}));
    if (mode == KFMI_MODE_UNFUSED) KFMI_TRY(check_ptrs({{qn, "qn"}}));
    if (vt) KFMI_TRY(check_ptrs({{vt, "vt"}}));
  }
  if ((cos == nullptr) != (sin == nullptr)) return fail(KFMI_EINVAL, "provide both rotary tables or neither");
  if (cos) KFMI_TRY(check_ptrs({{cos, "cos"}, {sin, "sin"}}));
  if (!(scale > 0.0)) return fail(KFMI_EINVAL, "scale must be > 0");
  KFMI_TRY(check_tuning(Hq, Hkv, D, mode == KFMI_MODE_FULL));
  KFMI_TRY(check_device());
  int64_t clear_bytes = 0;
  if (noalloc) {
    // A plan larger than the static array runs unsplit (no workspace), as
    // kfmi_launch_attention_bf16 does when given none.
    const int64_t need = kfmi::attention_workspace_bytes(B, Hq, Hkv, S, D, causal != 0);
    work = nullptr;
    work_bytes = 0;
    if (need > 0 && need <= KFMI_SCRATCH_BYTES) {
      hipError_t e = kfmi::noalloc_scratch(&work);
      if (e != hipSuccess) return launch_status(e, "static scratch address");
      work_bytes = KFMI_SCRATCH_BYTES;
      clear_bytes = kfmi::attention_workspace_counter_bytes(B, Hq, Hkv, S, D, causal != 0);
    }
  }
  hipStream_t st = (hipStream_t)stream;
  if (clear_bytes > 0) {  // the arrival counters start each launch at zero
    hipError_t e = kfmi::clear_scratch_words(work, clear_bytes, st);
    if (e != hipSuccess) return launch_status(e, "scratch clear launch");
  }
  if (mode == KFMI_MODE_FULL) {  // one launch, K normalised per tile; no scratch (rope:671-677)
    return attention_impl(q, k, v, nullptr, gq, gk, cos, sin, out, nullptr, B, Hq, Hkv, S, D, scale, eps, causal,
                          cos ? kfmi::PRO_NORM_ROPE : kfmi::PRO_NORM, style_of(norm_style), bm, bn, st, work,
                          work_bytes);
  }
  const bool rope = cos != nullptr;
  // V^T is used by the ping-pong kernel when its rows are 16-byte aligned.
  const bool use_vt = vt != nullptr && kfmi::attention_kernel(B, Hq, Hkv, S, D, causal != 0, false) == KFMI_KERNEL_PINGPONG && S % 8 == 0;
  kfmi::RowsArgs r{};
  r.q = (const uint16_t *)q; r.k = (const uint16_t *)k; r.gq = (const uint16_t *)gq; r.gk = (const uint16_t *)gk;
  r.cos = (const uint16_t *)cos; r.sin = (const uint16_t *)sin; r.qn = (uint16_t *)qn; r.kn = (uint16_t *)kn;
  r.B = B; r.Hq = Hq; r.Hkv = Hkv; r.S = S; r.D = D;
  r.only_k = mode == KFMI_MODE_QUERY; r.rope = rope; r.style = style_of(norm_style); r.eps = eps;
  if (use_vt) {  // the preparation launch also writes V^T
    r.v = (const uint16_t *)v;
    r.vt = (uint16_t *)vt;
  }
  hipError_t e = kfmi::launch_rows(r, st);
  if (e != hipSuccess) return launch_status(e, "prepare launch");
  const bool query = mode == KFMI_MODE_QUERY;
  const int pro = !query ? kfmi::PRO_NONE : (rope ? kfmi::PRO_NORM_ROPE : kfmi::PRO_NORM);
  return attention_impl(query ? q : qn, kn, v, use_vt ? vt : nullptr, gq, nullptr, cos, sin, out, nullptr, B, Hq, Hkv, S, D,
                        scale, eps, causal, pro, style_of(norm_style), bm, bn, st, work, work_bytes);
}

int kfmi_launch_attention_bf16(const void *q, const void *k, const void *v, const void *gq, const void *gk,
                               const void *cos, const void *sin, void *out, void *qn, void *kn, void *vt, int64_t B,
                               int64_t Hq, int64_t Hkv, int64_t S, int64_t D, double scale, float eps, int causal,
                               int mode, int norm_style, int bm, int bn, void *work, int64_t work_bytes,
                               void *stream) {
  return launch_attention_entry(q, k, v, gq, gk, cos, sin, out, qn, kn, vt, B, Hq, Hkv, S, D, scale, eps, causal,
                                mode, norm_style, bm, bn, work, work_bytes, stream, false);
}

int kfmi_launch_attention_bf16_noalloc(const void *q, const void *k, const void *v, const void *gq, const void *gk,
                                       const void *cos, const void *sin, void *out, void *qn, void *kn, void *vt,
                                       int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t D, double scale,
                                       float eps, int causal, int mode, int norm_style, int bm, int bn,
                                       void *stream) {
  return launch_attention_entry(q, k, v, gq, gk, cos, sin, out, qn, kn, vt, B, Hq, Hkv, S, D, scale, eps, causal,
                                mode, norm_style, bm, bn, nullptr, 0, stream, true);
}

int kfmi_transpose_v_bf16(const void *v, void *vt, int64_t BH, int64_t S, int64_t D, void *stream) {
  if (BH < 1 || S < 1) return fail(KFMI_EINVAL, "BH and S must be >= 1");
  if (D != 128 && D != 256) return fail(KFMI_EINVAL, "D must be 128 or 256 (got %lld)", (long long)D);
  if (S % 8 != 0) return fail(KFMI_EINVAL, "S must be a multiple of 8 (got %lld)", (long long)S);
  if (BH * S * D >= ((int64_t)1 << 31)) return fail(KFMI_EINVAL, "tensors must have fewer than 2^31 elements");
  KFMI_TRY(check_ptrs({{v, "v"}, {vt, "vt"}}));
  KFMI_TRY(check_device());
  return launch_status(kfmi::launch_transpose_v((const uint16_t *)v, (uint16_t *)vt, BH, S, D, (hipStream_t)stream),
                       "V transpose launch");
}

int kfmi_factored_prepare_bf16(const void *q, const void *k, const void *gq, const void *gk, float *inv, void *kn,
                               int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t D, float eps, void *stream) {
  KFMI_TRY(check_shape(B, Hq, Hkv, S, D));
  KFMI_TRY(check_ptrs({{q, "q"}, {k, "k"}, {gq, "gq"}, {gk, "gk"}, {inv, "inv"}, {kn, "kn"}}));
  if (!(eps >= 0.0f)) return fail(KFMI_EINVAL, "eps must be >= 0");
  KFMI_TRY(check_device());
  kfmi::RowsArgs r{};
  r.q = (const uint16_t *)q; r.k = (const uint16_t *)k; r.gq = (const uint16_t *)gq; r.gk = (const uint16_t *)gk;
  r.kn = (uint16_t *)kn; r.inv = inv;
  r.B = B; r.Hq = Hq; r.Hkv = Hkv; r.S = S; r.D = D;
  r.only_k = false; r.rope = false; r.style = kfmi::ST_FACTORED; r.eps = eps;
  return launch_status(kfmi::launch_rows(r, (hipStream_t)stream), "factored prepare launch");
}

int kfmi_factored_attention_bf16(const void *q, const void *kn, const void *v, float *inv, void *out, int64_t B,
                                 int64_t Hq, int64_t Hkv, int64_t S, int64_t D, float eps, int causal, int inv_mode,
                                 int bm, int bn, void *work, int64_t work_bytes, void *stream) {
  KFMI_TRY(check_shape(B, Hq, Hkv, S, D));
  KFMI_TRY(check_tiles(bm, bn));
  KFMI_TRY(check_work(work, work_bytes));
  KFMI_TRY(check_ptrs({{q, "q"}, {kn, "kn"}, {v, "v"}, {out, "out"}}));
  if (inv_mode != 0 && inv_mode != 1) return fail(KFMI_EINVAL, "inv_mode must be 0 (read) or 1 (compute)");
  if (inv_mode == 0) KFMI_TRY(check_ptrs({{inv, "inv"}}));
  if (inv && (reinterpret_cast<uintptr_t>(inv) & 3u)) return fail(KFMI_EINVAL, "inv must be 4-byte aligned");
  KFMI_TRY(check_tuning(Hq, Hkv, D, false));
  KFMI_TRY(check_device());
  const int pro = inv_mode == 0 ? kfmi::PRO_FACTORED_READ : kfmi::PRO_FACTORED_CALC;
  return attention_impl(q, kn, v, nullptr, nullptr, nullptr, nullptr, nullptr, out, inv, B, Hq, Hkv, S, D, 0.0, eps, causal, pro,
                        kfmi::ST_FP32, bm, bn, (hipStream_t)stream, work, work_bytes);
}

int kfmi_launch_factored_attention_bf16(const void *q, const void *k, const void *v, const void *gq, const void *gk,
                                        void *out, float *inv, void *kn, int64_t B, int64_t Hq, int64_t Hkv,
                                        int64_t S, int64_t D, float eps, int causal, int bm, int bn, void *work,
                                        int64_t work_bytes, void *stream) {
  KFMI_TRY(check_shape(B, Hq, Hkv, S, D));
  KFMI_TRY(check_tiles(bm, bn));
  KFMI_TRY(check_work(work, work_bytes));
  KFMI_TRY(check_ptrs({{q, "q"}, {k, "k"}, {v, "v"}, {gq, "gq"}, {gk, "gk"}, {out, "out"}, {inv, "inv"}, {kn, "kn"}}));
  if (!(eps >= 0.0f)) return fail(KFMI_EINVAL, "eps must be >= 0");
  KFMI_TRY(check_tuning(Hq, Hkv, D, false));
  KFMI_TRY(check_device());
  kfmi::RowsArgs r{};
  r.q = (const uint16_t *)q; r.k = (const uint16_t *)k; r.gq = (const uint16_t *)gq; r.gk = (const uint16_t *)gk;
  r.kn = (uint16_t *)kn; r.inv = inv;
  r.B = B; r.Hq = Hq; r.Hkv = Hkv; r.S = S; r.D = D;
  r.only_k = true; r.rope = false; r.style = kfmi::ST_FACTORED; r.eps = eps;
  hipError_t e = kfmi::launch_rows(r, (hipStream_t)stream);
  if (e != hipSuccess) return launch_status(e, "factored prepare launch");
  return attention_impl(q, kn, v, nullptr, nullptr, nullptr, nullptr, nullptr, out, inv, B, Hq, Hkv, S, D, 0.0, eps, causal,
                        kfmi::PRO_FACTORED_CALC, kfmi::ST_FP32, bm, bn, (hipStream_t)stream, work, work_bytes);
}

}  // extern "C"
