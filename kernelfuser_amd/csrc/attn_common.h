#pragma once
// Shared device code of the attention kernels (attention.hip: the general
// kernel and the dispatch; attn_pp.hip: the ping-pong kernel; attn_wide.hip:
// the wide-wave kernel): launch parameters, the Q prologue, the online
// softmax, GEMM helpers on v_mfma_f32_32x32x16_bf16, LDS tile staging and the
// epilogue.  Each kernel file includes it and compiles on its own.
//
// Causal / non-causal GQA flash-attention prefill on gfx950 bf16 MFMA with a
// fused Q prologue.  Counterpart of the reference's attention_v2_kernel
// (src/e1_rope_publication_v1.py:608-649) and factored_attention_kernel
// (src/e1_qk_publication_v3.py:612-638).
//
// The kernels sharing this arithmetic:
//   attn_pp_kernel   D=128, Hq/Hkv even (the Qwen3 shapes).  One workgroup =
//                    8 waves = two Q heads of one GQA group x 128 query rows,
//                    or, when Hq/Hkv is a multiple of 4, four heads x 64 rows.
//                    Waves w and w+4 run on the same SIMD; group A (waves 0-3,
//                    first head or heads) and group B (waves 4-7) alternate
//                    phase by phase between an MFMA phase (GEMM1 of tile t and
//                    GEMM2 of tile t-1) and a VALU phase (softmax of tile t),
//                    so on every SIMD one wave keeps the matrix core busy while
//                    the other computes exponentials.  Each K/V tile staged in
//                    LDS serves every head of the workgroup.
//   attn_fwd_kernel  any D in {128, 256} and GQA ratio: 4 waves = 128 query
//                    rows of one head; GEMM1 of tile t+1 is issued ahead of the
//                    softmax and GEMM2 of tile t.
//   attn_ww_kernel   D=128, Hq/Hkv a multiple of 4, on request only: 4 waves,
//                    one per SIMD, each holding 64 query rows of one head and
//                    pipelining GEMM1, softmax and GEMM2 of consecutive tiles
//                    inside itself (its file describes it).
//
// Transposed formulation (everything stays in registers between the GEMMs):
//   GEMM1  S^T = K . Q^T   A = K tile rows from LDS (ds_read_b128),
//                           B = the wave's 32 Q rows, held in VGPRs as MFMA
//                               B-operands for the whole sweep;
//          the 32x32 accumulator gives every lane ONE query (lane % 32) and 16
//          keys, so the row max / row sum are lane-local plus one
//          v_permlane32_swap with the other half-wave, and the per-query
//          rescale of O is a per-lane scalar;
//   GEMM2  O^T = V^T . P^T A = V^T read from the row-major V tile in LDS with
//                               ds_read_b64_tr_b16 (transpose on read), or,
//                               when the caller supplies V transposed per head
//                               (written by the preparation launch), from a
//                               V^T tile with one ds_read_b128 per operand,
//                           B = P^T straight from the GEMM1 accumulator
//                               (exp2, cvt to bf16, no data movement; with
//                               V^T the keys of each 16-key step are put in
//                               consecutive order by one v_permlane32_swap).
// MFMA: v_mfma_f32_32x32x16_bf16.  Operand layouts: A[m][k] -> lane
// m + 32*(k/8), element k%8; B[k][n] -> lane n + 32*(k/8), element k%8;
// C[m][n] -> lane n + 32*((m/4)%2), register (m/8)*4 + m%4.
//
// K/V staging: tiles of BN rows (16 KiB each) are copied HBM -> LDS by the
// buffer unit (buffer_load_dwordx4 ... lds: lane L of a copy writes LDS bytes
// base + 16*L), so no VGPRs, no ds_write and no bounds branches are spent on
// staging: each copy's full byte offset is its VGPR offset, which the raw-buffer
// range check covers, and the descriptor spans exactly one head's S rows, so
// rows past S arrive as zeros (never the next head's or another allocation's
// bytes).  Both K and V are double-buffered; the 16-byte chunks of each row are
// XOR-swizzled (K: chunk ^ (row & 15); V: chunk ^ 4*(row & 3)) so that the 16
// lanes of a GEMM1 row read (16 B each) and the 32 lanes of a GEMM2 transpose
// read (8 B each) cover all 64 LDS banks exactly once.
//
// Q prologue (query fusion): the wave's raw Q rows are loaded straight into
// the B-operand layout (lane: row lane%32, columns 16c + 8*(lane/32) + 0..7),
// where both rotate-half partners (d, d +/- D/2) sit in the same lane; the
// RMS needs one cross-half sum.  RMSNorm * gamma and RoPE run in FP32 with
// the rounding points of the selected style, then round once to BF16.
//
// Softmax: exp2 online softmax with scale*log2(e) folded into one FMA per
// score (rope:636-643).  The running max is raised only when a row's tile max
// exceeds it by more than 2^8 (log2 domain) -- probabilities then stay below
// 256, far inside FP32/BF16 range, and O is rescaled a handful of times per
// row instead of on every tile; after the final division by the row sum the
// result is the same softmax.  Causal: the KV loop stops at the diagonal,
// masks are applied only on diagonal/tail tiles, and the grid issues the
// longest query blocks first.
#include <math.h>

#include <atomic>

#include <cstdio>
#include <string>

#include "kfmi_device.h"
#include "kfmi_launch.h"

namespace kfmi {

struct AttnParams {
  const uint16_t *q, *k, *v, *gq, *cos, *sin;
  const uint16_t *gk;  // K's gamma for the per-tile K prologue (mode 'full'), else NULL
  const uint16_t *vt;  // V transposed per head ([B,Hkv,D,S]) for the VT kernels
  uint16_t *out;
  float *inv;
  int64_t S;
  int B, Hq, Hkv, n_qblocks, xcd_remap;
  // ping-pong kernel, persistent mode: number of (long, short) query-block
  // pairs; 0 = one item per workgroup
  int pp_units;
  // ping-pong kernel: Q heads per wave group (1: two heads x 128 query rows
  // per item; 2: four heads x 64 rows, for GQA ratios divisible by 4)
  int pp_hpg;
  // general kernel, causal, one round of two workgroups per CU (slot2 = the
  // CU count, > 0): workgroups bid and bid + slot2 share a CU, so the second
  // slot takes the query blocks shortest first and each CU's pair sums to
  // the same number of key tiles
  int slot2;
  float c_scale;  // scale*log2(e); for the factored prologues D^-1/2*log2(e)
  float eps;
  // Split-KV plan of the general kernel (n_items > 0): work item r of the
  // longest-first list covers query block it_qb[r] and key tiles
  // [it_t0[r], it_t1[r]); it_sid[r] >= 0 marks one half of split block
  // it_sid[r], whose partial results meet in `partials` and are merged by the
  // half that finishes second (decided by `counters`, which end each launch
  // at zero again).
  int n_items;
  int16_t it_qb[128], it_t0[128], it_t1[128], it_sid[128];
  int *counters;
  float *partials;
  // 4 * KFMI_CLOCK_STAMPS_MAX words of clock stamps, or NULL (no stamps)
  unsigned long long *stamps;
};
constexpr int MAX_SPLIT_ITEMS = 128;

// Clock stamps {t0, t1, r0, r1} of workgroup blockIdx.x (kfmi_clock_stamp):
// the shader-clock counter and the 100 MHz real-time counter, read by the
// first thread at the workgroup's start (END = false) and at each of its
// exits (END = true).  Vector stores to a device array; nothing when the
// launch passes no array.
template <bool END>
__device__ __forceinline__ void clock_stamp(unsigned long long *st) {
  if (st != nullptr && threadIdx.x == 0 && blockIdx.x < KFMI_CLOCK_STAMPS_MAX) {
    unsigned long long *e = st + 4 * blockIdx.x;
    e[END ? 1 : 0] = __builtin_amdgcn_s_memtime();
    e[END ? 3 : 2] = __builtin_amdgcn_s_memrealtime();
  }
}

namespace {


template <int ST>
__device__ __forceinline__ float norm_elem(float x, float inv, float g) {
  if (ST == ST_HF) return round_bf16(round_bf16(x * inv) * g);
  if (ST == ST_LEGACY) return round_bf16(__fmul_rn(__fmul_rn(x, inv), g));
  return __fmul_rn(__fmul_rn(x, inv), g);
}
template <int ST>
__device__ __forceinline__ float rope_elem(float n, float np, float c, float s, bool first) {
  if (ST == ST_FP32) {
    // No contraction into an FMA: both products are rounded, then the sum
    // (HIP's __fmul_rn/__fadd_rn are plain * and + that the headers let the
    // compiler contract, so the operators are written here).
#pragma clang fp contract(off)
    const float p0 = n * c, p1 = np * s;
    return first ? p0 - p1 : p0 + p1;
  }
  float p0 = round_bf16(n * c), p1 = round_bf16(np * s);
  return first ? p0 - p1 : p0 + p1;
}

__device__ __forceinline__ bf16x8_t as_bf16x8(const u32x4_t &w) { return __builtin_bit_cast(bf16x8_t, w); }

typedef int i32x4_t __attribute__((ext_vector_type(4)));

// Buffer descriptor of a byte range: raw addressing, reads at or past `bytes`
// return zeros.
__device__ __forceinline__ i32x4_t buffer_rsrc(const void *base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  i32x4_t r;
  r[0] = (int)(uint32_t)a;
  r[1] = (int)(uint32_t)(a >> 32);  // stride 0
  r[2] = (int)bytes;
  r[3] = 0x00020000;
  return r;
}

// 16 bytes per lane from buffer byte offset voff into LDS at lds + 16*lane.
// The whole offset travels in the VGPR operand (the SGPR offset is the
// constant 0): the raw-buffer range check compares voffset + the instruction
// offset with num_records, so a chunk at or past the descriptor's size reads
// as zeros whatever the hardware does with a non-zero SGPR offset.
// Issued as inline assembly so the compiler does not guard every later LDS
// read with a wait for it; the kernels order copies and reads themselves
// (wait_copies + barrier).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"  // m0 is reserved; it is set right here
__device__ __forceinline__ void copy16_to_lds(const i32x4_t &rsrc, uint32_t lds, uint32_t voff) {
  // lds is wave-uniform; readfirstlane pins it to an SGPR.
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(voff), "s"(rsrc)
               : "memory", "m0");
}
#pragma clang diagnostic pop

// Wait until every copy this wave issued has landed in LDS.
__device__ __forceinline__ void wait_copies() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

constexpr float RESCALE_SLACK = 8.0f;  // log2 units: probabilities stay <= 2^8
// Lean-softmax guard: a lane's partial sum of one tile's probabilities must
// stay below 2^64, so every probability does and O accumulates far inside
// FP32 range; otherwise the work item is redone with the exact softmax.
constexpr float FAST_LIMIT = 0x1p64f;

// Phase fences: an empty volatile asm that takes the phase's results as
// inputs, so the compiler finishes computing them before the barrier that
// ends the phase instead of sinking that work into the next phase.
// (The asm operands only exist in the device pass; the host pass of this
// file never executes device code.)
template <int N>
__device__ __forceinline__ void fence_regs(const f32x16_t (&x)[N]) {
#if defined(__HIP_DEVICE_COMPILE__)
#pragma unroll
  for (int i = 0; i < N; ++i) asm volatile("" ::"v"(x[i]));
#endif
}
template <int N>
__device__ __forceinline__ void fence_regs(const bf16x8_t (&x)[N]) {
#if defined(__HIP_DEVICE_COMPILE__)
#pragma unroll
  for (int i = 0; i < N; ++i) asm volatile("" ::"v"(x[i]));
#endif
}
__device__ __forceinline__ void fence_regs(float x) {
#if defined(__HIP_DEVICE_COMPILE__)
  asm volatile("" ::"v"(x));
#endif
}
// Phase entry: the registers count as rewritten here, so no work that reads
// them is hoisted above the barrier that starts the phase.
template <int N>
__device__ __forceinline__ void fence_in(f32x16_t (&x)[N]) {
#if defined(__HIP_DEVICE_COMPILE__)
#pragma unroll
  for (int i = 0; i < N; ++i) asm volatile("" : "+v"(x[i]));
#endif
}
template <int N>
__device__ __forceinline__ void fence_in(bf16x8_t (&x)[N]) {
#if defined(__HIP_DEVICE_COMPILE__)
#pragma unroll
  for (int i = 0; i < N; ++i) asm volatile("" : "+v"(x[i]));
#endif
}

// Source offset (bytes, from the first row of the tile) of the chunk that
// copy `inst` places in LDS slot lane%CPR of row inst*RPI + lane/CPR, for the
// K or V swizzle.  The caller adds the tile's own row offset.
template <int D>
__device__ __forceinline__ uint32_t copy_lane_offset(int inst, int lane, bool v_tile) {
  constexpr int RB = 2 * D, CPR = D / 8, RPI = 1024 / RB;
  const int row = inst * RPI + lane / CPR;
  const int slot = lane % CPR;
  const int chunk = v_tile ? (slot ^ ((row & 3) << 2)) : (slot ^ (row & 15));
  return (uint32_t)(row * RB + (chunk << 4));
}

// Per-lane LDS read offsets.  GEMM1: lane reads row 32*kb + lr, chunk 2c + g;
// with the K swizzle the slot is 16*(c/8) + ((2*(c%8) + g) ^ (lr & 15)), so
// kra[c%8] + 256*(c/8).  GEMM2 transpose reads: the 16-lane group supplies rows
// (lane%16)/4 + 4g of a 16-key step and 4-column runs 16*((lane/16)%2) +
// 4*(lane%4) of a 32-wide d block, i.e. chunk 4*db + 2*hh + kk; with the V
// swizzle (row % 4 = m) the slot is 16*(db/4) + 4*((db%4) ^ m) + 2*hh + kk, so
// vra[db%4] + 256*(db/4).
template <int D>
__device__ __forceinline__ void lds_read_offsets(int lane, uint32_t (&kra)[8], uint32_t (&vra)[4]) {
  constexpr int RB = 2 * D;
  const int g = lane >> 5, lr = lane & 31;
#pragma unroll
  for (int j = 0; j < 8; ++j) kra[j] = (uint32_t)(lr * RB + (((2 * j + g) ^ (lr & 15)) << 4));
  const int m = (lane >> 2) & 3, hh = (lane >> 4) & 1, kk = (lane >> 1) & 1;
  const int row0 = ((lane & 15) >> 2) + 4 * g;
#pragma unroll
  for (int e = 0; e < 4; ++e) vra[e] = (uint32_t)(row0 * RB + ((4 * (e ^ m) + 2 * hh + kk) << 4) + (lane & 1) * 8);
}

// Q prologue: the lane's query row -> GEMM1 B operands (columns 16c + 8g ..
// +7), optionally RMSNorm * gamma (+ RoPE), and the lane's logit multiplier.
// FOLD (FP32 style with a norm prologue only): the logit multiplier is
// applied to the normalised FP32 row before its single rounding, so the MFMA
// yields scores already in log2 units and cl becomes 1.
// Rotary table rows staged in LDS by the caller (STAGED; otherwise read from
// global memory): the lane's chunk 2c+g of cos is at cos + off[c], of sin at
// sin + off[c]; the copies are waited for at the barrier inside q_prologue.
// STAGED is a template parameter, not a null test of tab.cos, so that the
// unused global-load path is not compiled in (its loads, though never
// executed, made the compiler add waits for them).
struct StagedTables {
  const unsigned char *cos = nullptr, *sin = nullptr;
  const uint32_t *off = nullptr;
};

struct NoOp {
  __device__ void operator()() const {}
};

// after_tab() runs once the staged table rows are in registers (after a
// barrier), before the normalisation and rotation arithmetic.
template <int D, int PRO, int ST, bool FOLD = false, bool STAGED = false, typename AfterTab = NoOp>
__device__ __forceinline__ void q_prologue(const AttnParams &p, int64_t qoff, int qrow, bool qvalid, int g,
                                           bf16x8_t (&qreg)[D / 16], float &cl, const StagedTables tab = {},
                                           AfterTab after_tab = {}) {
  constexpr int NC = D / 16;
  const uint16_t *qbase = p.q + qoff * D;
  const u32x4_t zero = {0u, 0u, 0u, 0u};
  cl = p.c_scale;
  u32x4_t raw[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) raw[c] = qvalid ? ld16(qbase + (int64_t)qrow * D + 16 * c + 8 * g) : zero;
  if constexpr (PRO == PRO_NONE) {
    // The loaded rows are pinned as computed VGPR values (an empty asm that
    // rewrites them): left as plain loads, the general kernel's tile loop was
    // scheduled 28% slower in cycles at D=256 (84 against 66 us, Gemma-3-12B
    // B=1 S=2048) and 7% slower at D=128, with the same instruction counts.
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      qreg[c] = as_bf16x8(raw[c]);
      asm volatile("" : "+v"(qreg[c]));
    }
  } else if constexpr (PRO == PRO_FACTORED_READ) {
#pragma unroll
    for (int c = 0; c < NC; ++c) qreg[c] = as_bf16x8(raw[c]);
    cl = (qvalid ? p.inv[qoff + qrow] : 1.0f) * p.c_scale;  // qk:621
  } else {
    // gamma and the table rows are issued with the Q loads, so the prologue
    // waits for one round trip to memory, not two
    constexpr bool TAB = PRO == PRO_NORM_ROPE;
    constexpr bool GAM = PRO == PRO_NORM || PRO == PRO_NORM_ROPE;
    u32x4_t graw[GAM ? NC : 1], craw[TAB ? NC : 1], sraw[TAB ? NC : 1];
    if constexpr (GAM) {
#pragma unroll
      for (int c = 0; c < NC; ++c) graw[c] = ld16(p.gq + 16 * c + 8 * g);
    }
    if constexpr (TAB) {
      if constexpr (!STAGED) {
        const int64_t trow = qvalid ? (int64_t)qrow * D : 0;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          craw[c] = ld16(p.cos + trow + 16 * c + 8 * g);
          sraw[c] = ld16(p.sin + trow + 16 * c + 8 * g);
        }
      }
    }
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      float x[8];
      unpack8(raw[c], x);
#pragma unroll
      for (int j = 0; j < 8; ++j) ss = __fmaf_rn(x[j], x[j], ss);
    }
    ss = sum_halves(ss);
    const float inv = rsqrt_rn(ss * (1.0f / D) + p.eps);
    if constexpr (TAB) {
      if constexpr (STAGED) {
        wait_copies();
        __syncthreads();
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          craw[c] = *reinterpret_cast<const u32x4_t *>(tab.cos + tab.off[c]);
          sraw[c] = *reinterpret_cast<const u32x4_t *>(tab.sin + tab.off[c]);
        }
        after_tab();
      }
    }
    if constexpr (PRO == PRO_FACTORED_CALC) {
#pragma unroll
      for (int c = 0; c < NC; ++c) qreg[c] = as_bf16x8(raw[c]);
      if (p.inv != nullptr && g == 0 && qvalid) p.inv[qoff + qrow] = inv;  // qk:597-601
      cl = inv * p.c_scale;                                              // qk:621
    } else {
      constexpr int HC = NC / 2;  // chunk c pairs with c ^ HC (columns d, d + D/2)
#pragma unroll
      for (int c = 0; c < HC; ++c) {
        const int c2 = c + HC;
        float x1[8], x2[8], g1[8], g2[8], n1[8], n2[8], y1[8], y2[8];
        unpack8(raw[c], x1);
        unpack8(raw[c2], x2);
        unpack8(graw[c], g1);
        unpack8(graw[c2], g2);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          n1[j] = norm_elem<ST>(x1[j], inv, g1[j]);
          n2[j] = norm_elem<ST>(x2[j], inv, g2[j]);
        }
        if constexpr (PRO == PRO_NORM_ROPE) {
          float cs1[8], sn1[8], cs2[8], sn2[8];
          unpack8(craw[c], cs1);
          unpack8(sraw[c], sn1);
          unpack8(craw[c2], cs2);
          unpack8(sraw[c2], sn2);
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            y1[j] = rope_elem<ST>(n1[j], n2[j], cs1[j], sn1[j], true);
            y2[j] = rope_elem<ST>(n2[j], n1[j], cs2[j], sn2[j], false);
          }
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j) { y1[j] = n1[j]; y2[j] = n2[j]; }
        }
        if constexpr (FOLD) {
#pragma unroll
          for (int j = 0; j < 8; ++j) { y1[j] = __fmul_rn(y1[j], p.c_scale); y2[j] = __fmul_rn(y2[j], p.c_scale); }
        }
        qreg[c] = as_bf16x8(pack8(y1));
        qreg[c2] = as_bf16x8(pack8(y2));
      }
      if constexpr (FOLD) cl = 1.0f;
    }
  }
}

// Online-softmax state of one wave (32 query rows, one per lane pair).
//   FOLD = false: scores s are raw q.k; logits = s*cl (one FMA per score).
//   FOLD = true : GEMM1 starts from -m_run, so s already is logit - m_run
//                 (Q carries the multiplier); one exp2 per score.  m_run starts
//                 at 0 and the first tile always sets it to the exact row max.
//   CONSEC = false: P^T operand element j of half g is key
//                   16*c2 + 8*(j/4) + 4*g + j%4 (the accumulator's own order;
//                   matches the transpose reads of a row-major V tile);
//   CONSEC = true : element j of half g is key 16*c2 + 8*g + j (matches
//                   16-byte reads of V^T rows); two v_permlane32_swap per
//                   16-key step move the 4-key runs between the half-waves.
template <int D, int BN, bool CAUSAL, bool FOLD = false, bool CONSEC = false>
struct Softmax {
  static constexpr int NKB = BN / 32, NK16 = BN / 16, NDB = D / 32;
  float m_run = FOLD ? 0.f : -INFINITY;  // reference max of logits (log2 domain)
  float l_run = 0.f;                     // this lane's partial row sum
  bool started = false;                  // a tile has set m_run (FOLD and step_lean)

  // GEMM1 accumulator start value of this lane (FOLD: -m_run).
  __device__ __forceinline__ float acc_init() const { return FOLD ? -m_run : 0.f; }

  // Scores of KV tile t (keys t*BN ..) -> P^T operands pb; rescales o when
  // the reference max has to move.
  __device__ __forceinline__ void step(f32x16_t (&s)[NKB], int t, int q0, int qrow, int64_t S, int g, float cl,
                                       f32x16_t (&o)[NDB], bf16x8_t (&pb)[NK16]) {
    // masks: register i of block kb holds key kt + 4*g + c_i with the
    // compile-time c_i = 32*kb + 8*(i/4) + i%4; a key is masked when it lies
    // past the lane's query (causal) or past the sequence, i.e. when
    // c_i > lim = min(qrow, S - 1) - kt - 4*g.
    const int kt = t * BN;
    const bool need_mask = (CAUSAL && kt + BN - 1 > q0) || (kt + BN > S);
    if (need_mask) {
      const int last = (int)(S - 1);
      const int lim = (CAUSAL ? (qrow < last ? qrow : last) : last) - kt - 4 * g;
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (32 * kb + 8 * (i >> 2) + (i & 3) > lim) s[kb][i] = -INFINITY;
    }
    // Row max as a balanced tree (a serial chain would leave the VALU idle
    // on dependency latency).
    float mt[NKB * 8];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int i = 0; i < 8; ++i) mt[kb * 8 + i] = fmaxf(s[kb][2 * i], s[kb][2 * i + 1]);
#pragma unroll
    for (int n = NKB * 8; n > 1; n = (n + 1) / 2)  // fold the upper ceil half (NKB * 8 need not be 2^k)
#pragma unroll
      for (int i = 0; i + (n + 1) / 2 < n; ++i) mt[i] = fmaxf(mt[i], mt[i + (n + 1) / 2]);
    float ls[4] = {0.f, 0.f, 0.f, 0.f};  // four interleaved partial sums
    if constexpr (FOLD) {
      const float mx = max_halves(mt[0]);  // tile max of logit - m_run
      if (__builtin_amdgcn_ballot_w64(!started || mx > RESCALE_SLACK) != 0) {
        // First tile: m_run := row max; later: raise m_run by the excess.
        const float delta = started ? fmaxf(mx, 0.f) : mx;
        const float alpha = started ? __builtin_amdgcn_exp2f(-delta) : 0.f;
        l_run *= alpha;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
          for (int i = 0; i < 16; ++i) o[db][i] *= alpha;
        m_run += delta;
        started = true;
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
          for (int i = 0; i < 16; ++i) s[kb][i] -= delta;
      }
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float pv = __builtin_amdgcn_exp2f(s[kb][i]);
          s[kb][i] = pv;
          ls[i & 3] += pv;
        }
    } else {
      const float mx = max_halves(mt[0]) * cl;
      if (__builtin_amdgcn_ballot_w64(mx > m_run + RESCALE_SLACK) != 0) {
        const float m_new = fmaxf(m_run, mx);
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);  // 0 on the first tile
        l_run *= alpha;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
          for (int i = 0; i < 16; ++i) o[db][i] *= alpha;
        m_run = m_new;
      }
      const float neg_m = -m_run;
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kb][i], cl, neg_m));
          s[kb][i] = pv;
          ls[i & 3] += pv;
        }
    }
    l_run += (ls[0] + ls[1]) + (ls[2] + ls[3]);
    pack(s, pb);
  }

  // Lean tile (the general kernel's hot path).  The first tile of a sweep
  // (FIRST, peeled by the caller so later tiles carry no branch) sets m_run
  // to the tile's exact row max (O and l are still zero, so nothing is
  // rescaled); every later tile takes p = exp2(logit - m_run)
  // with no max reduction and no rescale.  That is the same softmax (one
  // constant shift per row), valid as long as no probability overflows:
  // a lane whose partial tile sum is not below FAST_LIMIT sets `bad` (rows
  // at or past S excluded), and the caller then redoes the whole work item
  // with step().  O never changes here, which keeps this path's register
  // footprint at that of the accumulators alone.
  template <bool FIRST>
  __device__ __forceinline__ void step_lean(f32x16_t (&s)[NKB], int t, int q0, int qrow, int64_t S, int g, float cl,
                                            bf16x8_t (&pb)[NK16], bool &bad) {
    const int kt = t * BN;
    const bool need_mask = (CAUSAL && kt + BN - 1 > q0) || (kt + BN > S);
    if (need_mask) {
      const int last = (int)(S - 1);
      const int lim = (CAUSAL ? (qrow < last ? qrow : last) : last) - kt - 4 * g;
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (32 * kb + 8 * (i >> 2) + (i & 3) > lim) s[kb][i] = -INFINITY;
    }
    if constexpr (FIRST) {
      float mt[NKB * 8];
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int i = 0; i < 8; ++i) mt[kb * 8 + i] = fmaxf(s[kb][2 * i], s[kb][2 * i + 1]);
#pragma unroll
      for (int n = NKB * 8; n > 1; n = (n + 1) / 2)
#pragma unroll
        for (int i = 0; i + (n + 1) / 2 < n; ++i) mt[i] = fmaxf(mt[i], mt[i + (n + 1) / 2]);
      const float mx = max_halves(mt[0]);
      if constexpr (FOLD) {
        m_run += mx;  // scores held logit - m_run with m_run = 0
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
          for (int i = 0; i < 16; ++i) s[kb][i] -= mx;
      } else {
        m_run = mx * cl;
      }
      started = true;
    }
    float ls[4] = {0.f, 0.f, 0.f, 0.f};
    const float nm = -m_run;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float pv = FOLD ? __builtin_amdgcn_exp2f(s[kb][i]) : __builtin_amdgcn_exp2f(__builtin_fmaf(s[kb][i], cl, nm));
        s[kb][i] = pv;
        ls[i & 3] += pv;
      }
    const float lt = (ls[0] + ls[1]) + (ls[2] + ls[3]);
    l_run += lt;
    bad |= qrow < S && !(lt < FAST_LIMIT);
    pack(s, pb);
  }

  // P^T operands: 16-key step c2 <- registers 8*(c2%2) .. +7 of block c2/2
  // (registers 4q..4q+3 of a block hold keys 8q + 4*g + 0..3).
  __device__ __forceinline__ void pack(const f32x16_t (&s)[NKB], bf16x8_t (&pb)[NK16]) const {
#pragma unroll
    for (int c2 = 0; c2 < NK16; ++c2) {
      u32x4_t wv;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        wv[j] = pack_bf16x2(s[c2 >> 1][8 * (c2 & 1) + 2 * j], s[c2 >> 1][8 * (c2 & 1) + 2 * j + 1]);
      if constexpr (CONSEC) {
        // half 0 keeps its keys 0-3 and takes the other half's 4-7; half 1
        // takes keys 8-11 and keeps its 12-15 (permlane32_swap(a, b) yields
        // [a_lo, b_lo] and [a_hi, b_hi]).
        const auto x0 = __builtin_amdgcn_permlane32_swap(wv[0], wv[2], false, false);
        const auto x1 = __builtin_amdgcn_permlane32_swap(wv[1], wv[3], false, false);
        wv[0] = x0[0];
        wv[1] = x1[0];
        wv[2] = x0[1];
        wv[3] = x1[1];
      }
      pb[c2] = as_bf16x8(wv);
    }
  }
};

// GEMM1: S^T (BN keys x 32 queries) of the K tile at LDS byte kbuf.
constexpr int G1_AHEAD = 2;
template <int D, int BN>
__device__ __forceinline__ void gemm1(const unsigned char *smem, int kbuf, const uint32_t (&kra)[8],
                                      const bf16x8_t (&qreg)[D / 16], f32x16_t (&s)[BN / 32]) {
  constexpr int RB = 2 * D, NKB = BN / 32, NC = D / 16;
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb) s[kb] = f32x16_t{};
#pragma unroll
  for (int c = 0; c < NC; ++c) {  // alternating accumulation chains
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      const bf16x8_t a = *reinterpret_cast<const bf16x8_t *>(smem + kbuf + kb * 32 * RB + kra[c & 7] + (c >> 3) * 256);
      s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qreg[c], s[kb], 0, 0, 0);
    }
  }
  // Issue order: K reads run G1_AHEAD MFMAs ahead, so an MFMA's operand was
  // requested several MFMAs (~32 cycles each) before it, past the LDS
  // latency.
  __builtin_amdgcn_sched_group_barrier(0x100, G1_AHEAD, 0);
#pragma unroll
  for (int i = 0; i < NKB * NC; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    if (i + G1_AHEAD < NKB * NC) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
  }
}

// GEMM1 with the K prologue of mode 'full' (rope:630-631, FUSE_K): the lane's
// raw K row chunks are read from the tile (row 32*kb + lr: columns 16c + 8g ..
// +7 for every c, both rotate-half partners d and d +/- D/2 in this lane),
// RMSNorm * gamma_k (+ RoPE at the key's position) is applied in FP32 with the
// style's rounding points, rounded to BF16, and the MFMAs use the result.
// The RMS needs one cross-half sum.  Keys past S are zero rows (their table
// row is clamped to 0); they are masked later.  Every wave recomputes the
// tile's rows, as every program of the reference does.
template <int D, int BN, int ST, bool ROPE>
__device__ __forceinline__ void gemm1_fused_k(const unsigned char *smem, int kbuf, const uint32_t (&kra)[8],
                                              const bf16x8_t (&qreg)[D / 16], f32x16_t (&s)[BN / 32],
                                              const AttnParams &p, int key0, int g, int lr) {
  constexpr int RB = 2 * D, NKB = BN / 32, NC = D / 16, HC = NC / 2;
  auto chunk = [&](int kb, int c) -> u32x4_t {
    return *reinterpret_cast<const u32x4_t *>(smem + kbuf + kb * 32 * RB + kra[c & 7] + (c >> 3) * 256);
  };
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb) {
    // pass 1: sum of squares of the row (chunks re-read in pass 2 instead of
    // being held, to keep the register footprint of the loop)
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      float x[8];
      unpack8(chunk(kb, c), x);
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) ss = __fmaf_rn(x[jj], x[jj], ss);
    }
    ss = sum_halves(ss);
    const float inv = rsqrt_rn(ss * (1.0f / D) + p.eps);
    const int key = key0 + 32 * kb + lr;
    const int64_t trow = key < p.S ? (int64_t)key * D : 0;
    // pass 2: one rotate-half pair (c, c + D/32 chunks) at a time; the MFMAs
    // accumulate in chunk order 0 .. NC-1, as in gemm1.
    bf16x8_t khi[HC];
    s[kb] = f32x16_t{};
#pragma unroll
    for (int c = 0; c < HC; ++c) {
      const int c2 = c + HC;
      float x1[8], x2[8], g1[8], g2[8], n1[8], n2[8], y1[8], y2[8];
      unpack8(chunk(kb, c), x1);
      unpack8(chunk(kb, c2), x2);
      unpack8(ld16(p.gk + 16 * c + 8 * g), g1);
      unpack8(ld16(p.gk + 16 * c2 + 8 * g), g2);
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) {
        n1[jj] = norm_elem<ST>(x1[jj], inv, g1[jj]);
        n2[jj] = norm_elem<ST>(x2[jj], inv, g2[jj]);
      }
      if constexpr (ROPE) {
        float cs1[8], sn1[8], cs2[8], sn2[8];
        unpack8(ld16(p.cos + trow + 16 * c + 8 * g), cs1);
        unpack8(ld16(p.sin + trow + 16 * c + 8 * g), sn1);
        unpack8(ld16(p.cos + trow + 16 * c2 + 8 * g), cs2);
        unpack8(ld16(p.sin + trow + 16 * c2 + 8 * g), sn2);
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
          y1[jj] = rope_elem<ST>(n1[jj], n2[jj], cs1[jj], sn1[jj], true);
          y2[jj] = rope_elem<ST>(n2[jj], n1[jj], cs2[jj], sn2[jj], false);
        }
      } else {
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) { y1[jj] = n1[jj]; y2[jj] = n2[jj]; }
      }
      s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(pack8(y1)), qreg[c], s[kb], 0, 0, 0);
      khi[c] = as_bf16x8(pack8(y2));
      // one pair at a time: the scheduler would otherwise hoist every table
      // load of the tile and run out of registers
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int c = 0; c < HC; ++c) s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(khi[c], qreg[c + HC], s[kb], 0, 0, 0);
  }
}

// GEMM2: O^T[d][query] += V^T . P^T for the V tile at LDS byte vbuf; the A
// operand's slot j of half g is key 16*c2 + 8*(j/4) + 4*g + j%4, matching the
// P^T registers of Softmax::step.
template <int D, int BN>
__device__ __forceinline__ void gemm2(const unsigned char *smem, int vbuf, const uint32_t (&vra)[4],
                                      const bf16x8_t (&pb)[BN / 16], f32x16_t (&o)[D / 32]) {
  constexpr int RB = 2 * D, NK16 = BN / 16, NDB = D / 32;
#pragma unroll
  for (int c2 = 0; c2 < NK16; ++c2) {
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      const unsigned char *base = smem + vbuf + 16 * c2 * RB + vra[db & 3] + (db >> 2) * 256;
      const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t *)(base));
      const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t *)(base + 8 * RB));
      const bf16x8_t a = __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
      o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pb[c2], o[db], 0, 0, 0);
    }
  }
  // Issue order: V^T reads (two per MFMA) run two MFMAs ahead.
  __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
  for (int i = 0; i < NK16 * NDB; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    if (i + 2 < NK16 * NDB) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
  }
}

// GEMM1 of one tile and GEMM2 of the previous tile as one straight-line block
// (the ping-pong kernel's MFMA phase).  Issue order: six reads ahead, one read
// after each GEMM1 MFMA, two after each GEMM2 MFMA, so every MFMA's operand
// was requested several MFMAs earlier.
//   VT = false: the V tile is row-major (keys x D); two transpose reads per
//               GEMM2 MFMA (vra offsets).
//   VT = true : the tile holds V^T rows (D rows x BN keys, 2*BN bytes each,
//               chunk ^ ((row >> 1) & 7) swizzle); one 16-byte read per GEMM2
//               MFMA: row 32*db + lr, chunk 2*c2 + g (vra[c2] + 32*db*2*BN).
template <int D, int BN, bool VT = false>
__device__ __forceinline__ void mfma_phase(const unsigned char *smem, int kbuf, int vbuf, const uint32_t (&kra)[8],
                                           const uint32_t (&vra)[4], const bf16x8_t (&qreg)[D / 16], float s0,
                                           f32x16_t (&s)[BN / 32], const bf16x8_t (&pb)[BN / 16],
                                           f32x16_t (&o)[D / 32]) {
  constexpr int RB = 2 * D, NKB = BN / 32, NC = D / 16, NK16 = BN / 16, NDB = D / 32;
  constexpr int M1 = NKB * NC, M2 = NK16 * NDB, READS = M1 + (VT ? 1 : 2) * M2, AHEAD = 6;
  // GEMM1: the key blocks' accumulation chains alternate, so consecutive
  // MFMAs never depend on each other
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
    for (int i = 0; i < 16; ++i) s[kb][i] = s0;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      const bf16x8_t a = *reinterpret_cast<const bf16x8_t *>(smem + kbuf + kb * 32 * RB + kra[c & 7] + (c >> 3) * 256);
      s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qreg[c], s[kb], 0, 0, 0);
    }
  }
#pragma unroll
  for (int c2 = 0; c2 < NK16; ++c2) {
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      bf16x8_t a;
      if constexpr (VT) {
        a = *reinterpret_cast<const bf16x8_t *>(smem + vbuf + db * 32 * 2 * BN + vra[c2]);
      } else {
        const unsigned char *base = smem + vbuf + 16 * c2 * RB + vra[db & 3] + (db >> 2) * 256;
        const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t *)(base));
        const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t *)(base + 8 * RB));
        a = __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
      }
      o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pb[c2], o[db], 0, 0, 0);
    }
  }
  int issued = AHEAD;
  __builtin_amdgcn_sched_group_barrier(0x100, AHEAD, 0);
#pragma unroll
  for (int i = 0; i < M1 + M2; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    const int want = (i < M1 || VT) ? 1 : 2;
    const int n = issued + want <= READS ? want : READS - issued;
    if (n == 2) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    if (n == 1) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    issued += n;
  }
}

// Epilogue: O = O^T / l as BF16 rows, stored from the registers (8-byte
// pieces of 32 rows per instruction; used where no LDS staging fits).
template <int D>
__device__ __forceinline__ void store_rows(uint16_t *obase, int qrow, bool qvalid, int g, float l_run,
                                           const f32x16_t (&o)[D / 32]) {
  const float l_tot = sum_halves(l_run);
  if (!qvalid) return;
  const float rl = __fdiv_rn(1.0f, l_tot);
  uint16_t *orow = obase + (int64_t)qrow * D;
#pragma unroll
  for (int db = 0; db < D / 32; ++db)
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      u32x2_t wv;
      wv[0] = pack_bf16x2(o[db][4 * q4 + 0] * rl, o[db][4 * q4 + 1] * rl);
      wv[1] = pack_bf16x2(o[db][4 * q4 + 2] * rl, o[db][4 * q4 + 3] * rl);
      *reinterpret_cast<u32x2_t *>(orow + 32 * db + 8 * q4 + 4 * g) = wv;
    }
}

// Epilogue: O = O^T / l as BF16 rows, staged through LDS.  The lane owning
// query row lr holds 4-column runs of it (columns 32*db + 8*q + 4*g + 0..3);
// they are written to a row-major tile of the wave's 32 rows (16-byte chunk
// k of row r in slot k ^ (r % CPR)) and read back as whole chunks, CPR lanes
// per row, so each global store instruction writes 64 / CPR contiguous rows
// instead of 8-byte pieces of 32 rows.  `tile` is 32 * 2D bytes of LDS that
// no other wave touches until the caller's next barrier.  Rows at or past S
// are not stored.
template <int D>
__device__ __forceinline__ void store_rows_lds(unsigned char *tile, uint16_t *obase, int q0, int64_t S, int lane,
                                               float l_run, const f32x16_t (&o)[D / 32]) {
  constexpr int RB = 2 * D, CPR = D / 8, RPI = 64 / CPR;
  const int lr = lane & 31, g = lane >> 5;
  const float l_tot = sum_halves(l_run);
  const float rl = __fdiv_rn(1.0f, l_tot);
#pragma unroll
  for (int db = 0; db < D / 32; ++db)
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      u32x2_t wv;
      wv[0] = pack_bf16x2(o[db][4 * q4 + 0] * rl, o[db][4 * q4 + 1] * rl);
      wv[1] = pack_bf16x2(o[db][4 * q4 + 2] * rl, o[db][4 * q4 + 3] * rl);
      const int k = 4 * db + q4;  // 16-byte chunk of columns 32*db + 8*q4 ..
      *reinterpret_cast<u32x2_t *>(tile + lr * RB + ((k ^ (lr % CPR)) << 4) + 8 * g) = wv;
    }
  // The wave reads back its own writes: the LDS executes one wave's accesses
  // in issue order, and this keeps the compiler from reordering them.
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  const int c = lane % CPR, rr = lane / CPR;
  constexpr int NB = 4;  // reads per batch, issued before the batch's row-guarded stores
#pragma unroll
  for (int i0 = 0; i0 < 32 / RPI; i0 += NB) {
    u32x4_t x[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int r = (i0 + i) * RPI + rr;
      x[i] = *reinterpret_cast<const u32x4_t *>(tile + r * RB + ((c ^ (r % CPR)) << 4));
    }
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int r = (i0 + i) * RPI + rr;
      if (q0 + r < S) st16(obase + (int64_t)(q0 + r) * D + 8 * c, x[i]);
    }
  }
}

// The bits of x as an integer the compiler cannot trace back to a float.  In
// files built without NaN semantics a test of the exponent bits of a value
// that comes from floating-point arithmetic is otherwise rewritten as a
// floating-point class test (fabs(x) == inf, unordered) whose operand is
// assumed not NaN, and a NaN then passes it.
__device__ __forceinline__ uint32_t opaque_bits(float x) {
  uint32_t u = __float_as_uint(x);
  asm("" : "+v"(u));
  return u;
}
__device__ __forceinline__ bool not_finite(float x) {
  return (opaque_bits(x) & 0x7f800000u) == 0x7f800000u;  // exponent field all ones: inf or NaN
}
// Any accumulator inf or NaN: the largest magnitude bit pattern is at least
// the exponent-all-ones pattern.  Integer arithmetic on one accumulator
// register: a floating-point sum of the values can be NaN (+inf + -inf),
// which code built without NaN semantics may assume away, and a class test
// per value takes a scalar register pair each.
template <int N>
__device__ __forceinline__ bool any_not_finite(const f32x16_t (&o)[N]) {
  uint32_t m[2] = {0u, 0u};
#pragma unroll
  for (int n = 0; n < N; ++n)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const uint32_t a = __float_as_uint(o[n][i]) & 0x7fffffffu;
      m[i & 1] = m[i & 1] > a ? m[i & 1] : a;
    }
  return (m[0] > m[1] ? m[0] : m[1]) >= 0x7f800000u;
}

}  // namespace

// Launchers of the kernels that live in their own files (runtime dispatch
// over the template instances of each file).
hipError_t launch_pp(const AttnParams &p, bool causal, int pro, int st, int blocks, hipStream_t s);
hipError_t launch_wide(const AttnParams &p, bool causal, int pro, int st, int blocks, hipStream_t s);

}  // namespace kfmi
