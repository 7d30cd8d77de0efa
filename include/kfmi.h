/*
 * kfmi.h -- C ABI of the MI355X (gfx950) RoPE-aware attention prologue.
 *
 * The drop-in boundary for KernelFuser's attention-prologue path
 * (WenbinWang12/KernelFuser).  The reference has no native boundary: its
 * Python launchers start Triton kernels on torch's current stream.  Each entry
 * point below replaces one of those launchers and names the reference
 * function (file:line) whose launch it takes over.  References:
 *   rope = src/e1_rope_publication_v1.py, qk = src/e1_qk_publication_v3.py.
 *
 * Conventions (all entry points):
 *   - BF16 tensors are passed as raw device pointers to contiguous row-major
 *     data in the reference layout: Q/out [B,Hq,S,D], K/V/KN [B,Hkv,S,D],
 *     gamma [D], rotary tables [S,D] (split-half, duplicated halves), INV
 *     float32 [B,Hq,S].  Pointers must be 16-byte aligned.
 *   - D is 128 or 256; Hq % Hkv == 0; every tensor has < 2^31 elements
 *     (rope:708-717).
 *   - The caller owns every buffer.  No entry point allocates, frees or
 *     synchronises; all work is enqueued on `stream` (a hipStream_t, NULL =
 *     the legacy default stream), so calls are graph-capturable.
 *   - Return value: KFMI_OK, or an error code with a message available from
 *     kfmi_last_error() (thread-local).  Argument errors are detected before
 *     any launch, so a failing call enqueues nothing.
 */
#ifndef KFMI_H
#define KFMI_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KFMI_ABI_VERSION 10

/* status codes */
#define KFMI_OK 0
#define KFMI_EINVAL 1  /* invalid argument (shape, pointer, mode) */
#define KFMI_ELAUNCH 2 /* HIP launch or runtime error */
#define KFMI_EDEVICE 3 /* current device is not gfx950 */

/* norm_style (rope:680-681, :697-698, :559-563); FP32 = single final rounding,
 * the FP32 semantics of rope:119-130 (transform_debug). */
#define KFMI_NORM_HF 0
#define KFMI_NORM_LEGACY 1
#define KFMI_NORM_FP32 2

/* flags of kfmi_prepare_bf16 */
#define KFMI_PREP_ONLY_K 1 /* rope:591-595 ONLY_K */
#define KFMI_PREP_ROPE 2   /* rope:564 ROPE */

/* mode of kfmi_launch_attention_bf16 (rope:668) */
#define KFMI_MODE_QUERY 0   /* K prepared once, Q norm(+RoPE) in the attention prologue */
#define KFMI_MODE_UNFUSED 1 /* Q and K prepared, plain attention */
#define KFMI_MODE_FULL 2    /* one launch: Q and K norm(+RoPE) inside attention, K per key tile */

/* attention kernels (kfmi_tuning.attn_kernel, kfmi_launch_info.kernel) */
#define KFMI_KERNEL_AUTO 0     /* chosen by shape */
#define KFMI_KERNEL_GENERAL 1  /* attn_fwd_kernel: 4 waves x 32 rows of one head, D 128 or 256 */
#define KFMI_KERNEL_PINGPONG 2 /* attn_pp_kernel: 8 waves, two wave groups alternating MFMA and softmax phases */
#define KFMI_KERNEL_WIDE 3     /* attn_ww_kernel: 4 waves x 64 rows, four heads of a GQA group per item */

/* Version of this ABI (KFMI_ABI_VERSION). */
int kfmi_abi_version(void);

/* Message of the last failing call on this thread ("" if none). */
const char *kfmi_last_error(void);

/* One kernel launched by an entry-point call (see kfmi_last_launches). */
typedef struct {
  char kernel[96];       /* kernel instance, e.g. "attn_pp_kernel<true, 2, 2, false>" */
  int64_t grid;          /* workgroups */
  int32_t block;         /* threads per workgroup */
  int32_t registers;     /* registers per thread (hipFuncGetAttributes numRegs) */
  int32_t lds_bytes;     /* static LDS per workgroup */
  int32_t scratch_bytes; /* private memory per thread (register spills) */
  char plan[64];         /* choices made at launch time, "key=value" separated by spaces:
                            attention: "hpg=<Q heads per wave group> persistent=<0|1> xcd=<0|1>"
                            (ping-pong, wide) or "split=<query blocks split in two> pair=<0|1>
                            xcd=<0|1>" (general); rows: "hpw=<heads per workgroup>" */
} kfmi_launch_info;

/* The kernels launched by this thread's last successful compute call, in
 * launch order: copies up to `max` records into `out` (may be NULL when max
 * is 0) and returns how many that call launched (0 before any, or after a
 * call that failed before launching).  Replaces the kernel objects that the
 * reference's launchers return (launch_attention rope:674-677,
 * launch_factored_attention qk:651), whose consumer reads registers, spills
 * and shared memory (fusion_harness.py:82-102 compiler_evidence). */
int kfmi_last_launches(kfmi_launch_info *out, int max);

/* Dispatch choices that the library otherwise makes by shape, for tuning
 * runs: the counterpart of the Triton tile arguments (bm, bn, warps, stages,
 * gather) that the reference's tuning runner sweeps (tune_refinement,
 * rope:765-814).  Settings apply to later calls of the calling thread only;
 * a field left at 0 keeps the shape-based choice.  A forced choice that
 * cannot run a call's shape makes that call fail with KFMI_EINVAL before
 * anything is launched.  Results never depend on these settings beyond
 * last-bit differences of the kernels' own summation orders. */
typedef struct {
  int32_t attn_kernel; /* KFMI_KERNEL_*; modes other than FULL (FULL always runs the general kernel) */
  int32_t pp_heads;    /* ping-pong kernel: Q heads per wave group, 1 (two heads x 128 rows per
                          item) or 2 (four heads x 64 rows; GQA ratio a multiple of 4) */
  int32_t rows_heads;  /* preparation kernel: heads per workgroup for Q+K launches at D = 128,
                          2 or 4 (4 only without V^T and outside the factored preparation) */
  int32_t split;       /* general kernel at D = 256: 1 never splits a query block's key range */
  int32_t persistent;  /* ping-pong and wide kernels: 1 = one work item per workgroup (no
                          persistent long/short pairing) */
  int32_t clock_stamps; /* 1 = attention launches record per-workgroup clock stamps
                           (kfmi_clock_stamps); results are unchanged */
} kfmi_tuning;

/* Set (t != NULL) or clear (t == NULL) the calling thread's overrides.
 * Returns KFMI_EINVAL for out-of-range fields.  No counterpart in the
 * reference (see kfmi_tuning). */
int kfmi_set_tuning(const kfmi_tuning *t);

/* The calling thread's current overrides (all zero unless set). */
void kfmi_get_tuning(kfmi_tuning *out);

/* Clock stamps of one attention workgroup: the shader-clock counter
 * (s_memtime) and the 100 MHz real-time counter (s_memrealtime), read by the
 * workgroup's first thread when it starts (t0, r0) and when it ends (t1, r1).
 * (t1 - t0) / (r1 - r0) * 100 MHz is the workgroup's average shader clock. */
typedef struct {
  uint64_t t0, t1, r0, r1;
} kfmi_clock_stamp;

#define KFMI_CLOCK_STAMPS_MAX 2048 /* workgroups past this record none */

/* Stamps of the last attention launch that recorded them (kfmi_tuning
 * .clock_stamps = 1) on the current device: waits for the device, copies up
 * to `max` entries (one per workgroup, in workgroup order) into `out` (may be
 * NULL when max is 0) and returns how many that launch recorded (0 before
 * any), or -KFMI_EINVAL / -KFMI_EDEVICE / -KFMI_ELAUNCH.  Every recording launch on a GPU writes that GPU's one static array
 * (KFMI_CLOCK_STAMPS_MAX entries, held until the process ends), so launches
 * that record at the same time on one GPU race on it.  No counterpart in the
 * reference: it measures the clock that bounds a kernel's MFMA rate, which
 * the GPU lowers under power limits. */
int kfmi_clock_stamps(kfmi_clock_stamp *out, int max);

/* Row preparation: per-(token,head) RMSNorm(eps) * gamma, then optional
 * rotate-half RoPE, BF16 out.  Replaces prepare_attention -> prepare_kernel
 * (rope:652-658, :585-605, row math :550-582).  Q rows are skipped when
 * flags has KFMI_PREP_ONLY_K (q and qn may then be NULL); cos/sin are read
 * only when flags has KFMI_PREP_ROPE.  Also serves the isolated Q/K norm+RoPE
 * workload (Q and K rows in one launch).
 * vt (may be NULL; then v is ignored): the same launch also writes V
 * transposed per head, vt[b,h,d,s] = v[b,h,s,d] (D == 128, S % 8 == 0) -- the
 * V^T operand of kfmi_attention_bf16.  This addition has no counterpart in
 * the reference, whose kernels read V directly. */
int kfmi_prepare_bf16(const void *q, const void *k, const void *v, const void *gq, const void *gk,
                      const void *cos, const void *sin, void *qn, void *kn, void *vt,
                      int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t D,
                      float eps, int norm_style, int flags, void *stream);

/* Causal/non-causal GQA flash-attention prefill on bf16 MFMA.  Replaces the
 * attention_v2_kernel launch (rope:674-677, kernel :608-649).
 *   fuse_q = 1: q is raw; its RMSNorm (gq, eps, norm_style) and, when cos/sin
 *               are non-NULL, RoPE run in the kernel prologue (FUSE_Q=True).
 *   fuse_q = 0: q is already prepared (FUSE_Q=False).
 * k must be prepared (KN).  scale multiplies q.k (the reference uses D^-1/2,
 * rope:676).  bm is the number of query rows per workgroup (multiple of 32;
 * 128 is the tuned value), bn the key tile (64 or 128; a scheduling hint,
 * results do not depend on it).  vt (optional, may be NULL): V transposed per
 * head ([B,Hkv,D,S], as written by kfmi_prepare_bf16 or kfmi_transpose_v_bf16);
 * used instead of v under the conditions given at kfmi_launch_attention_bf16. */
int kfmi_attention_bf16(const void *q, const void *k, const void *v, const void *vt, const void *gq,
                        const void *cos, const void *sin, void *out,
                        int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t D,
                        double scale, float eps, int causal, int fuse_q, int norm_style,
                        int bm, int bn, void *work, int64_t work_bytes, void *stream);

/* Bytes of the optional split-KV workspace `work` of the attention entry
 * points for this shape (0: the shape never splits; -1: invalid shape).
 * For causal D = 256 shapes with no more query blocks than the GPU has CUs
 * (that kernel runs one workgroup per CU), the key range of the longest
 * query blocks is split over two workgroups whose partial results are merged
 * by the one finishing second; the workspace holds a 4 KiB region of
 * arrival counters (the same for every shape) followed by those partials.
 * The caller zero-fills it once when allocating; each launch leaves the
 * counters at zero again, so one workspace serves any sequence of shapes
 * that fit in it.  Calls that share a workspace must not overlap in time.
 * With work == NULL or work_bytes below this size the launch does not split
 * (same results, slower on those shapes).  No counterpart in the reference,
 * whose launches never split a query block. */
int64_t kfmi_attention_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t D, int causal);

/* The attention kernel (KFMI_KERNEL_GENERAL, _PINGPONG or _WIDE) that an
 * attention call of this shape and mode (KFMI_MODE_*) launches on the
 * current device under the calling thread's overrides (kfmi_set_tuning);
 * -KFMI_EINVAL for an invalid shape or mode, or overrides that cannot run
 * it.  Launches nothing.  No counterpart in the reference, whose launchers
 * always run their one Triton kernel. */
int kfmi_attention_kernel(int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t D, int causal, int mode);

/* The launches of launch_attention (rope:661-677): mode QUERY prepares K
 * into kn (K rows only) then runs attention with the fused Q prologue; mode
 * UNFUSED prepares Q into qn and K into kn, then runs plain attention; mode
 * FULL is one launch in which attention normalises (and rotates) Q in its
 * prologue and every K tile as it uses it (FUSE_Q and FUSE_K, rope:619-635;
 * qn, kn and vt are unused and may be NULL).  gk is K's gamma.  Scratch kn
 * (and qn for UNFUSED) is caller-allocated, as the reference requires
 * (rope:665-672).  cos/sin NULL disables RoPE.
 * vt (optional, may be NULL): caller-allocated scratch of V's size; when
 * given, the shape runs the ping-pong kernel (kfmi_attention_kernel) and
 * S % 8 == 0, the preparation launch
 * also writes V transposed per head ([B,Hkv,D,S]) and the attention kernel
 * reads that instead of V (one 16-byte LDS read per V operand instead of two
 * transposing 8-byte reads).  Results are identical either way; the call
 * stays two launches. */
int kfmi_launch_attention_bf16(const void *q, const void *k, const void *v,
                               const void *gq, const void *gk, const void *cos,
                               const void *sin, void *out, void *qn, void *kn, void *vt,
                               int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t D,
                               double scale, float eps, int causal, int mode,
                               int norm_style, int bm, int bn, void *work, int64_t work_bytes,
                               void *stream);

/* kfmi_launch_attention_bf16 without the work/work_bytes arguments, for
 * callers that cannot allocate (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  No counterpart in the reference,
 * whose launches never split a query block and so need no workspace.  The
 * split-KV workspace of the causal D = 256 shapes that split (see
 * kfmi_attention_workspace_bytes) is a static device array of 36 MiB per GPU
 * (held by each GPU the library runs on until the process ends); a shape
 * whose split plan needs more runs unsplit, exactly as
 * kfmi_launch_attention_bf16 with no workspace (results within a few ulp of
 * the split launch's).  The call allocates nothing: when the shape splits it enqueues a
 * small fill kernel that zeroes the plan's arrival counters ahead of the
 * other launches.  Every call on one GPU shares that GPU's array, so calls
 * that overlap in time on one GPU (several streams, or concurrent graph
 * replays) race on it.  Results are identical to kfmi_launch_attention_bf16
 * with a zero-filled caller workspace (with none, for the plans that do not
 * fit). */
int kfmi_launch_attention_bf16_noalloc(const void *q, const void *k, const void *v,
                                       const void *gq, const void *gk, const void *cos,
                                       const void *sin, void *out, void *qn, void *kn, void *vt,
                                       int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t D,
                                       double scale, float eps, int causal, int mode,
                                       int norm_style, int bm, int bn, void *stream);

/* vt[b,h,d,s] = v[b,h,s,d] for B*H heads of S rows of D (D 128 or 256,
 * S % 8 == 0): the V^T scratch of kfmi_launch_attention_bf16, as a separate
 * launch.  No counterpart in the reference (its kernels read V directly). */
int kfmi_transpose_v_bf16(const void *v, void *vt, int64_t BH, int64_t S, int64_t D, void *stream);

/* Factored no-RoPE preparation (qk:592-609): INV[B,Hq,S] = rsqrt(mean q^2 +
 * eps) (float32) for every Q row and KN = bf16(k * inv_k * gk * gq) for every
 * K row (one rounding). */
int kfmi_factored_prepare_bf16(const void *q, const void *k, const void *gq, const void *gk,
                               float *inv, void *kn, int64_t B, int64_t Hq, int64_t Hkv,
                               int64_t S, int64_t D, float eps, void *stream);

/* Factored attention (qk:612-638): scores = (q_raw . kn) * inv[row] * D^-1/2
 * with exp2 online softmax; q is the RAW (un-normalised) BF16 query.
 * inv_mode = 0: read inv (written by kfmi_factored_prepare_bf16);
 * inv_mode = 1: compute each row's inverse RMS from q in the prologue
 * (eps) and also write it to inv (which may then be NULL to skip the write).
 * work / work_bytes: the optional split-KV workspace, as for
 * kfmi_launch_attention_bf16 (same plan, same kfmi_attention_workspace_bytes;
 * NULL runs unsplit). */
int kfmi_factored_attention_bf16(const void *q, const void *kn, const void *v, float *inv,
                                 void *out, int64_t B, int64_t Hq, int64_t Hkv, int64_t S,
                                 int64_t D, float eps, int causal, int inv_mode, int bm, int bn,
                                 void *work, int64_t work_bytes, void *stream);

/* Both launches of launch_factored_attention (qk:641-652): KN preparation
 * for the K rows, then factored attention that computes INV in its prologue
 * and writes it to inv.  Outputs out, inv and kn match the reference's.
 * work / work_bytes: the optional split-KV workspace of the attention launch
 * (as for kfmi_launch_attention_bf16; NULL runs unsplit).  The reference's
 * launcher takes none. */
int kfmi_launch_factored_attention_bf16(const void *q, const void *k, const void *v,
                                        const void *gq, const void *gk, void *out, float *inv,
                                        void *kn, int64_t B, int64_t Hq, int64_t Hkv, int64_t S,
                                        int64_t D, float eps, int causal, int bm, int bn,
                                        void *work, int64_t work_bytes, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* KFMI_H */
