// Causal / non-causal GQA flash-attention prefill on gfx950 bf16 MFMA with a
// fused Q prologue.  Counterpart of the reference's attention_v2_kernel
// (src/e1_rope_publication_v1.py:608-649) and factored_attention_kernel
// (src/e1_qk_publication_v3.py:612-638).
//
// Two kernels share the arithmetic below:
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
namespace {

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
};
constexpr int MAX_SPLIT_ITEMS = 128;

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
#pragma unroll
    for (int c = 0; c < NC; ++c) qreg[c] = as_bf16x8(raw[c]);
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

// ---------------------------------------------------------------------------
// Ping-pong kernel: D=128, BN=64, two or four Q heads of a GQA group per
// workgroup.  With four (p.pp_hpg = 2) each item covers 64 query rows, so
// that no wave of a causal item runs a key tile that is masked for all of its
// rows (with 128-row items, waves holding the block's first 64 rows do at the
// diagonal), and the staged table rows halve.
// ---------------------------------------------------------------------------
template <bool CAUSAL, int PRO, int ST, bool VT>
__global__ __launch_bounds__(512, 1) void attn_pp_kernel(AttnParams p) {
  constexpr int D = 128, BN = 64, BM = 128;
  constexpr int TILE = BN * 2 * D;      // 16 KiB
  constexpr int LPW = TILE / 1024 / 8;  // copies per wave per tile (2)
  constexpr int NC = D / 16, NDB = D / 32, NKB = BN / 32, NK16 = BN / 16;
  constexpr int K0 = 0, K1 = TILE, V0 = 2 * TILE, V1 = 3 * TILE;
  // Rotary table rows of the block's BM positions (cos, then sin), shared by
  // both heads: staged with coalesced copies instead of 32 rows per load.
  constexpr int TROWS = 4 * TILE, TAB_BYTES = BM * 2 * D;
  constexpr bool STAGE_TAB = PRO == PRO_NORM_ROPE;

  __shared__ __attribute__((aligned(1024))) unsigned char smem[4 * TILE + (STAGE_TAB ? 2 * TAB_BYTES : 0)];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // 0..7
  const int grp = w >> 2;  // 0: first head (group A), 1: second head (group B)
  const int wq = w & 3;    // 32-row block of the workgroup's 128 rows
  const int g = lane >> 5;
  const int lr = lane & 31;
  const int64_t S = p.S;

  const int G = p.Hq / p.Hkv;
  const int hpg = p.pp_hpg;     // Q heads per wave group
  const int BMI = BM / hpg;     // query rows per item
  const int HP = G / (2 * hpg);  // items of one query block per KV head (head pairs or quads)
  const int npairs = p.B * p.Hkv * HP;
  // wave's head within the item's 2*hpg heads and its 32-row block
  const int hsub = grp * hpg + (hpg == 2 ? (wq >> 1) : 0);
  const int rblk = hpg == 2 ? (wq & 1) : wq;
  const uint32_t lds0 = (uint32_t)reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) unsigned char *)smem);

  // One work item: query block qb (BMI rows) of head pair (or quad) j of KV
  // head kvi.
  auto run = [&](const int qb, const int kvi, const int j) {
  const int b = kvi / p.Hkv;
  const int kvh = kvi - b * p.Hkv;
  const int h = kvh * G + 2 * hpg * j + hsub;
  const int64_t qoff = ((int64_t)b * p.Hq + h) * S;
  const int64_t kvoff = ((int64_t)b * p.Hkv + kvh) * S;

  const uint32_t head_bytes = (uint32_t)(S * 2 * D);
  const i32x4_t krs = buffer_rsrc(p.k + kvoff * D, head_bytes);
  const i32x4_t vrs = buffer_rsrc((VT ? p.vt : p.v) + kvoff * D, head_bytes);
  uint32_t kvo[LPW], vvo[LPW];
#pragma unroll
  for (int i = 0; i < LPW; ++i) {
    const int inst = w * LPW + i;
    kvo[i] = copy_lane_offset<D>(inst, lane, false);
    if constexpr (VT) {
      // VT tile: copy inst fills V^T rows 8*inst + lane/8 (2*BN = 128 bytes of
      // keys each), slot lane%8, swizzle chunk ^ ((row >> 1) & 7).
      const int row = 8 * inst + lane / 8;
      vvo[i] = (uint32_t)(row * S * 2 + (((lane % 8) ^ ((row >> 1) & 7)) << 4));
    } else {
      vvo[i] = copy_lane_offset<D>(inst, lane, true);
    }
  }
  auto copy_k = [&](int t, int buf) {
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
      const int inst = w * LPW + i;
      copy16_to_lds(krs, lds0 + buf + inst * 1024, kvo[i] + (uint32_t)(t * TILE));
    }
  };
  auto copy_v = [&](int t, int buf) {
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
      const int inst = w * LPW + i;
      copy16_to_lds(vrs, lds0 + buf + inst * 1024, vvo[i] + (uint32_t)(VT ? t * 2 * BN : t * TILE));
    }
  };

  const int q0 = qb * BMI + rblk * 32;
  const int qrow = q0 + lr;
  const bool qvalid = qrow < S;
  const int64_t kv_end = CAUSAL ? ((int64_t)(qb + 1) * BMI < S ? (int64_t)(qb + 1) * BMI : S) : S;
  const int nT = (int)((kv_end + BN - 1) / BN);

  copy_k(0, K0);

  uint32_t kra[8], vra[4];
  lds_read_offsets<D>(lane, kra, vra);
  StagedTables tab;
  if constexpr (STAGE_TAB) {
    // wave w copies rows (BMI/8)w .. of each table, 4 rows per copy, with
    // the K tiles' chunk swizzle, so kra[c] addresses the lane's row chunk
    const i32x4_t crs = buffer_rsrc(p.cos, (uint32_t)(S * 2 * D));
    const i32x4_t srs = buffer_rsrc(p.sin, (uint32_t)(S * 2 * D));
    const int ncp = 4 / hpg;
    for (int i = 0; i < ncp; ++i) {
      const int j = ncp * w + i;
      const uint32_t voff = copy_lane_offset<D>(j, lane, false) + (uint32_t)(qb * BMI * 2 * D);
      copy16_to_lds(crs, lds0 + TROWS + j * 1024, voff);
      copy16_to_lds(srs, lds0 + TROWS + TAB_BYTES + j * 1024, voff);
    }
    tab.cos = smem + TROWS + rblk * 32 * 2 * D;
    tab.sin = tab.cos + TAB_BYTES;
    tab.off = kra;
  }

  constexpr bool FOLD = ST == ST_FP32 && (PRO == PRO_NORM || PRO == PRO_NORM_ROPE);
  bf16x8_t qreg[NC];
  float cl;
  q_prologue<D, PRO, ST, FOLD, STAGE_TAB>(p, qoff, qrow, qvalid, g, qreg, cl, tab);
  if constexpr (VT) {
    // V^T reads: row 32*db + lr, chunk 2*c2 + g, swizzled by (row >> 1) & 7.
#pragma unroll
    for (int j = 0; j < 4; ++j) vra[j] = (uint32_t)(lr * 2 * BN + (((2 * j + g) ^ ((lr >> 1) & 7)) << 4));
  }

  f32x16_t o[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) o[db] = f32x16_t{};
  Softmax<D, BN, CAUSAL, FOLD, VT> sm;
  f32x16_t s[NKB];
  bf16x8_t pb[NK16];
#pragma unroll
  for (int c2 = 0; c2 < NK16; ++c2) pb[c2] = bf16x8_t{};
  {
    // Zero the V1 buffer read by M(0) (it is first filled in iteration 1).
    const u32x4_t z = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < TILE / (16 * 512); ++i) st16((uint16_t *)(smem + V1 + 16 * (tid + 512 * i)), z);
  }

  // Each wave runs M(0) V(0) M(1) V(1) ... V(nT-1) M(nT) with
  //   M(t) = GEMM1 of tile t (t < nT) + GEMM2 of tile t-1 (t >= 1),
  //   V(t) = softmax of tile t.
  // Group B runs one phase behind group A, so every phase pairs an M with a
  // V on each SIMD: iteration t = phase 2t (A: M(t), B: V(t-1)) and phase
  // 2t+1 (A: V(t), B: M(t)).  K(t+1) and V(t) are copied at the start of
  // phase 2t into the buffers that K(t-1) and V(t-2) left at the end of phase
  // 2t-1, and waited for at the start of phase 2t+2.  Both groups pass the
  // same two barriers per iteration; each group has its own straight-line
  // loop, and PAR = t % 2 selects the buffers at compile time.
  auto copies = [&](auto par, int t) {
    constexpr int PAR = decltype(par)::value;
    wait_copies();
    __syncthreads();
    if (t + 1 < nT) copy_k(t + 1, PAR ? K0 : K1);
    if (t < nT) copy_v(t, PAR ? V1 : V0);
  };
  // M(0)'s GEMM2 multiplies the zero P^T operands with the zero-filled V1
  // buffer and M(nT)'s GEMM1 reads a stale K buffer into scores nobody uses:
  // the MFMA phase is one straight-line block, so its LDS reads can run ahead
  // of the MFMAs that consume them across the GEMM1/GEMM2 boundary.
  auto mphase = [&](auto par, int t) {
    constexpr int PAR = decltype(par)::value;
    fence_in(pb);
    fence_in(o);
    mfma_phase<D, BN, VT>(smem, PAR ? K1 : K0, PAR ? V0 : V1, kra, vra, qreg, sm.acc_init(), s, pb, o);
    fence_regs(s);
    fence_regs(o);
  };
  auto vphase = [&](int t) {
    fence_in(s);
    fence_in(o);
    sm.step(s, t, q0, qrow, S, g, cl, o, pb);
    fence_regs(pb);
    fence_regs(o);
    fence_regs(sm.l_run);
  };
  if (grp == 0) {
    auto iter = [&](auto par, int t) {
      copies(par, t);
      mphase(par, t);
      __syncthreads();
      if (t < nT) vphase(t);
    };
    for (int t = 0;;) {
      iter(std::integral_constant<int, 0>{}, t);
      if (++t > nT) break;
      iter(std::integral_constant<int, 1>{}, t);
      if (++t > nT) break;
    }
  } else {
    auto iter = [&](auto par, int t) {
      copies(par, t);
      if (t >= 1) vphase(t - 1);
      __syncthreads();
      mphase(par, t);
    };
    for (int t = 0;;) {
      iter(std::integral_constant<int, 0>{}, t);
      if (++t > nT) break;
      iter(std::integral_constant<int, 1>{}, t);
      if (++t > nT) break;
    }
  }

  __syncthreads();  // both groups are past their last reads of the K/V buffers
  store_rows_lds<D>(smem + w * (32 * 2 * D), p.out + qoff * D, q0, S, lane, sm.l_run, o);
  };

  // ---- work items.  Persistent (pp_units > 0, causal): workgroup bid takes
  // units bid, bid + grid, ...; unit u pairs query blocks R-1-m and m of one
  // head pair (or quad), so every unit holds the same number of key tiles, and the
  // grid (a multiple of 8) keeps unit u on XCD u % 8, the home of its KV
  // head.  Otherwise one item per workgroup, heaviest blocks first.  Both
  // share one call site of `run`, so its body is emitted once. ----
  const int R = p.n_qblocks;
  int u = blockIdx.x, phase = 0;
  for (;;) {
    int qb, kvi, j;
    if (p.pp_units > 0) {
      if (u >= p.pp_units) break;
      const int per_kv = HP * ((R + 1) / 2);
      const int rest = u >> 3;
      kvi = (u & 7) + 8 * (rest / per_kv);
      const int rem = rest % per_kv;
      j = rem % HP;
      const int m = rem / HP;
      qb = phase == 0 ? R - 1 - m : m;
      if (phase == 0 && m != R - 1 - m) {
        phase = 1;
      } else {
        phase = 0;
        u += gridDim.x;
      }
    } else {
      if (u < 0) break;
      const int bid = u;
      u = -1;
      const int rank = bid / npairs;
      const int r = bid - rank * npairs;
      qb = CAUSAL ? R - 1 - rank : rank;
      if (p.xcd_remap) {
        // all head pairs of a KV head on one XCD so its K/V stay in that L2
        const int xcd = r & 7, jj = r >> 3;
        kvi = xcd + 8 * (jj / HP);
        j = jj % HP;
      } else {
        kvi = r / HP;
        j = r - kvi * HP;
      }
    }
    run(qb, kvi, j);
    __syncthreads();  // the next item refills the LDS buffers
  }
}

// ---------------------------------------------------------------------------
// General kernel: one head, 4 waves x 32 rows, D in {128, 256}.
// ---------------------------------------------------------------------------
template <int D, int BN, bool CAUSAL, int PRO, int ST, bool FK = false>
__global__ __launch_bounds__(256, (D == 128 ? 2 : 1)) void attn_fwd_kernel(AttnParams p) {
  // FK: K arrives raw and every tile gets the K prologue of mode 'full'.
  static_assert(!FK || PRO == PRO_NORM || PRO == PRO_NORM_ROPE, "mode 'full' fuses Q as well");
  constexpr int BM = 128;            // query rows per workgroup (4 waves x 32)
  constexpr int RB = 2 * D;          // bytes per K/V row
  constexpr int TILE = BN * RB;      // bytes per K or V tile
  constexpr int NINST = TILE / 1024; // 1 KiB copies per tile
  constexpr int LPW = NINST / 4;     // copies per wave per tile
  constexpr int NC = D / 16, NKB = BN / 32, NK16 = BN / 16, NDB = D / 32;
  constexpr int K0 = 0, K1 = TILE, V0 = 2 * TILE, V1 = 3 * TILE;
  static_assert(TILE == 16384 && LPW * 4 == NINST, "tiles are 16 KiB, 4 copies per wave");

  __shared__ __attribute__((aligned(1024))) unsigned char smem[4 * TILE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5;   // half-wave: selects k-group of the MFMA operands
  const int lr = lane & 31;  // query row of this lane within the wave
  const int64_t S = p.S;

  // ---- work item: heaviest query blocks (or split halves) first; KV groups
  // pinned to an XCD ----
  const int nbh = p.B * p.Hq;
  const int bid = blockIdx.x;
  const int rank = bid / nbh;
  const int r = bid - rank * nbh;
  int qb, t0 = 0, t1 = -1, sid = -1;
  if (p.n_items > 0) {
    qb = p.it_qb[rank];
    t0 = p.it_t0[rank];
    t1 = p.it_t1[rank];
    sid = p.it_sid[rank];
  } else if (CAUSAL && p.slot2 > 0 && bid >= p.slot2) {
    qb = (bid - p.slot2) / nbh;
  } else {
    qb = CAUSAL ? p.n_qblocks - 1 - rank : rank;
  }
  const int G = p.Hq / p.Hkv;
  int b, h;
  if (p.xcd_remap) {
    // Workgroups are dispatched round-robin over the 8 XCDs (bid % 8).  Map
    // KV group kg to XCD kg % 8 so the G query heads that read the same K/V
    // share one L2.
    const int xcd = r & 7, jj = r >> 3;
    const int kg = xcd + 8 * (jj / G);
    b = kg / p.Hkv;
    h = (kg - b * p.Hkv) * G + jj % G;
  } else {
    b = r / p.Hq;
    h = r - b * p.Hq;
  }
  const int kvh = h / G;
  const int64_t qoff = ((int64_t)b * p.Hq + h) * S;
  const int64_t kvoff = ((int64_t)b * p.Hkv + kvh) * S;

  const uint32_t head_bytes = (uint32_t)(S * RB);
  const i32x4_t krs = buffer_rsrc(p.k + kvoff * D, head_bytes);
  const i32x4_t vrs = buffer_rsrc(p.v + kvoff * D, head_bytes);
  const uint32_t lds0 = (uint32_t)reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) unsigned char *)smem);
  uint32_t kvo[LPW], vvo[LPW];
#pragma unroll
  for (int i = 0; i < LPW; ++i) {
    kvo[i] = copy_lane_offset<D>(w * LPW + i, lane, false);
    vvo[i] = copy_lane_offset<D>(w * LPW + i, lane, true);
  }
  auto copy_k = [&](int t, int buf) {
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
      const int inst = w * LPW + i;
      copy16_to_lds(krs, lds0 + buf + inst * 1024, kvo[i] + (uint32_t)(t * TILE));
    }
  };
  auto copy_v = [&](int t, int buf) {
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
      const int inst = w * LPW + i;
      copy16_to_lds(vrs, lds0 + buf + inst * 1024, vvo[i] + (uint32_t)(t * TILE));
    }
  };

  const int q0 = qb * BM + w * 32;
  const int qrow = q0 + lr;
  const bool qvalid = qrow < S;

  // ---- KV tile range [t0, nT) of this work item ----
  const int64_t kv_end = CAUSAL ? ((int64_t)(qb + 1) * BM < S ? (int64_t)(qb + 1) * BM : S) : S;
  const int nT = t1 >= 0 ? t1 : (int)((kv_end + BN - 1) / BN);
  const int64_t wave_end = CAUSAL ? ((int64_t)q0 + 32 < S ? (int64_t)q0 + 32 : S) : S;
  const int nTw0 = q0 < S ? (int)((wave_end + BN - 1) / BN) : 0;  // tiles with any unmasked key
  const int nTw = nTw0 < nT ? nTw0 : nT;

  uint32_t kra[8], vra[4];
  lds_read_offsets<D>(lane, kra, vra);

  auto first_copies = [&]() {
    copy_k(t0, K0);
    copy_v(t0, V0);
    if (t0 + 1 < nT) copy_k(t0 + 1, K1);
  };
  // D = 128 with RoPE: the rotary-table rows of the wave's 32 positions are
  // first staged in the K/V buffers (cos in the first 32 KiB, sin in the
  // second) with coalesced copies (8 per table per wave, the K tiles' chunk
  // swizzle, so kra[c] addresses the lane's chunks) instead of loads that
  // each touch 32 rows.  Once every wave holds its rows in registers the
  // first K/V copies are issued; they land while the prologue computes.
  constexpr bool STAGE_TAB = D == 128 && PRO == PRO_NORM_ROPE && !FK;
  StagedTables tab;
  if constexpr (STAGE_TAB) {
    const i32x4_t crs = buffer_rsrc(p.cos, (uint32_t)(S * RB));
    const i32x4_t srs = buffer_rsrc(p.sin, (uint32_t)(S * RB));
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int j = 8 * w + i;  // rows 4j .. 4j+3 of the block
      const uint32_t voff = copy_lane_offset<D>(j, lane, false) + (uint32_t)(qb * BM * RB);
      copy16_to_lds(crs, lds0 + j * 1024, voff);
      copy16_to_lds(srs, lds0 + 32768 + j * 1024, voff);
    }
    tab.cos = smem + w * 32 * RB;
    tab.sin = tab.cos + 32768;
    tab.off = kra;
  } else {
    // Start the first copies before the prologue's own global loads.
    first_copies();
  }

  bf16x8_t qreg[NC];
  float cl;
  if constexpr (STAGE_TAB) {
    q_prologue<D, PRO, ST, false, true>(p, qoff, qrow, qvalid, g, qreg, cl, tab, [&]() {
      __syncthreads();  // every wave's table reads have completed
      first_copies();
    });
  } else {
    q_prologue<D, PRO, ST>(p, qoff, qrow, qvalid, g, qreg, cl);
  }

  f32x16_t o[NDB];
  Softmax<D, BN, CAUSAL> sm;
  bool bad = false;  // a lean tile of this lane failed its overflow guard

  // Pipeline (one barrier per KV tile): iteration t issues the copies of
  // K(t+2) and V(t+1), then GEMM1 of tile t+1 and the softmax + GEMM2 of tile
  // t; each copy has a full iteration to land.  PAR = t % 2 selects buffers;
  // LEAN selects Softmax::step_lean (hot path) or Softmax::step (exact).
  auto iteration = [&](auto par, auto lean, auto first, int t, f32x16_t (&cur)[NKB], f32x16_t (&nxt)[NKB]) {
    constexpr int PAR = decltype(par)::value;
    constexpr bool LEAN = decltype(lean)::value;
    constexpr bool FIRST = decltype(first)::value;
    constexpr int KNEXT = PAR ? K0 : K1;   // holds K(t+1)
    constexpr int KFREE = PAR ? K1 : K0;   // held K(t), read in the previous iteration
    constexpr int VCUR = PAR ? V1 : V0;    // holds V(t)
    constexpr int VFREE = PAR ? V0 : V1;   // held V(t-1)
    wait_copies();
    __syncthreads();
    if (t + 2 < nT) copy_k(t + 2, KFREE);
    if (t + 1 < nT) copy_v(t + 1, VFREE);
    if (t + 1 < nTw) {
      if constexpr (FK)
        gemm1_fused_k<D, BN, ST, PRO == PRO_NORM_ROPE>(smem, KNEXT, kra, qreg, nxt, p, (t + 1) * BN, g, lr);
      else
        gemm1<D, BN>(smem, KNEXT, kra, qreg, nxt);
    }
    if (t < nTw) {
      bf16x8_t pb[NK16];
      if constexpr (LEAN)
        sm.template step_lean<FIRST>(cur, t, q0, qrow, S, g, cl, pb, bad);
      else
        sm.step(cur, t, q0, qrow, S, g, cl, o, pb);
      gemm2<D, BN>(smem, VCUR, vra, pb, o);
    }
  };
  // One sweep over the work item's KV tiles; the first K/V copies must have
  // been issued.
  auto sweep = [&](auto lean) {
#pragma unroll
    for (int db = 0; db < NDB; ++db) o[db] = f32x16_t{};
    sm = Softmax<D, BN, CAUSAL>{};
    f32x16_t sa[NKB], sb[NKB];
    wait_copies();
    __syncthreads();
    if (t0 < nTw) {
      if constexpr (FK)
        gemm1_fused_k<D, BN, ST, PRO == PRO_NORM_ROPE>(smem, K0, kra, qreg, sa, p, t0 * BN, g, lr);
      else
        gemm1<D, BN>(smem, K0, kra, qreg, sa);
    }
    // the first tile is peeled (it alone reduces the row max on the lean path)
    iteration(std::integral_constant<int, 0>{}, lean, std::true_type{}, t0, sa, sb);
    for (int t = t0 + 1; t < nT;) {
      iteration(std::integral_constant<int, 1>{}, lean, std::false_type{}, t, sb, sa);
      if (++t >= nT) break;
      iteration(std::integral_constant<int, 0>{}, lean, std::false_type{}, t, sa, sb);
      ++t;
    }
  };
  if constexpr (FK) {
    sweep(std::false_type{});  // mode 'full' runs at the register limit: exact path only
  } else {
    sweep(std::true_type{});
    // A lean tile failed somewhere in the workgroup (a logit far above the
    // first tile's row max): every wave redoes the item on the exact path.
    if (__syncthreads_or(bad)) {
      first_copies();
      sweep(std::false_type{});
    }
  }

  // the host plans splits for D = 256 only (plan_split)
  if (D != 256 || sid < 0) {
    if constexpr (FK) {
      // mode 'full' runs at the register limit: direct stores
      store_rows<D>(p.out + qoff * D, qrow, qvalid, g, sm.l_run, o);
    } else {
      __syncthreads();  // the K/V buffers become the epilogue's staging tiles
      store_rows_lds<D>(smem + w * (32 * 2 * D), p.out + qoff * D, q0, S, lane, sm.l_run, o);
    }
    return;
  }
  // ---- one half of a split query block: publish the partial state (O
  // relative to m_run, the lane's row-sum share, m_run); the half that
  // finishes second reads the other's, merges and stores, and re-arms the
  // counter.  Slot layout (floats): O quad q of thread tid at
  // [(q * 256 + tid) * 4], m_run at [NQ * 1024 + tid], l_run after it.
  //
  // The slots are written and read with agent-coherent accesses (cache
  // policy SC1, what the compiler gives agent-scope atomic accesses on
  // gfx950): a store that has completed (vmcnt) is visible to SC1 loads on
  // any XCD.  That orders the handover through the counter without the L2
  // writeback and invalidate that a device-scope fence costs.
  constexpr int NQ = NDB * 4;
  constexpr int SLOT = (NQ * 4 + 2) * 256;  // floats
  constexpr int SC1 = 16;
  const int part = t0 > 0 ? 1 : 0;
  // wave-uniform (sid, b, h are per workgroup): keeps the descriptors in SGPRs
  const int pair = __builtin_amdgcn_readfirstlane(sid * nbh + (b * p.Hq + h));
  const auto mine =
      __builtin_amdgcn_make_buffer_rsrc(p.partials + (int64_t)(2 * pair + part) * SLOT, 0, SLOT * 4, 0x00020000);
  const auto other =
      __builtin_amdgcn_make_buffer_rsrc(p.partials + (int64_t)(2 * pair + 1 - part) * SLOT, 0, SLOT * 4, 0x00020000);
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const f32x4_t v = {o[q / 4][(q % 4) * 4], o[q / 4][(q % 4) * 4 + 1], o[q / 4][(q % 4) * 4 + 2],
                       o[q / 4][(q % 4) * 4 + 3]};
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, v), mine, (q * 256 + tid) * 16, 0, SC1);
  }
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, sm.m_run), mine, (NQ * 1024 + tid) * 4, 0, SC1);
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, sm.l_run), mine, (NQ * 1024 + 256 + tid) * 4, 0,
                                        SC1);
  wait_copies();  // every store of this thread has completed
  __syncthreads();
  __shared__ int arrived_before;
  if (tid == 0) {
    // Release/acquire at agent scope around the arrival counter (the
    // memory model's own mapping: L2 writeback before, invalidate after), so
    // the handover is ordered even where the SC1 accesses alone would not
    // be; one thread per workgroup, after the barrier that follows every
    // thread's completed stores.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    arrived_before = atomicAdd(p.counters + pair, 1);
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  }
  __syncthreads();
  if (arrived_before == 0) return;  // the other half merges
  // Merge in fixed (first half, second half) operand order, whichever half
  // runs it, with explicit fmaf, so the result does not depend on timing.
  const float mo = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(other, (NQ * 1024 + tid) * 4, 0, SC1));
  const float lo =
      __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(other, (NQ * 1024 + 256 + tid) * 4, 0, SC1));
  const float m0 = part == 0 ? sm.m_run : mo, m1 = part == 0 ? mo : sm.m_run;
  const float m = fmaxf(m0, m1);
  // rows past S may hold -inf maxima in both halves; they are not stored
  const float a0 = m0 == m ? 1.0f : __builtin_amdgcn_exp2f(m0 - m);
  const float a1 = m1 == m ? 1.0f : __builtin_amdgcn_exp2f(m1 - m);
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const f32x4_t v = __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(other, (q * 256 + tid) * 16, 0, SC1));
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float r = o[q / 4][(q % 4) * 4 + k];
      const float x0 = part == 0 ? r : v[k], x1 = part == 0 ? v[k] : r;
      o[q / 4][(q % 4) * 4 + k] = fmaf(x0, a0, x1 * a1);
    }
  }
  const float l0 = part == 0 ? sm.l_run : lo, l1 = part == 0 ? lo : sm.l_run;
  __syncthreads();
  store_rows_lds<D>(smem + w * (32 * 2 * D), p.out + qoff * D, q0, S, lane, fmaf(l0, a0, l1 * a1), o);
  if (tid == 0) atomicExch(p.counters + pair, 0);
}

// Launch-log names of the kernel instances (formatted once per instance).
template <int D, int BN, bool CAUSAL, int PRO, int ST, bool FK>
const char *fwd_name() {
  static const std::string n = [] {
    char b[96];
    snprintf(b, sizeof(b), "attn_fwd_kernel<%d, %d, %s, %d, %d, %s>", D, BN, tf(CAUSAL), PRO, ST, tf(FK));
    return std::string(b);
  }();
  return n.c_str();
}
template <bool CAUSAL, int PRO, int ST, bool VT>
const char *pp_name() {
  static const std::string n = [] {
    char b[96];
    snprintf(b, sizeof(b), "attn_pp_kernel<%s, %d, %d, %s>", tf(CAUSAL), PRO, ST, tf(VT));
    return std::string(b);
  }();
  return n.c_str();
}

template <int D, int BN, bool CAUSAL, int PRO, int ST>
hipError_t launch_t(const AttnParams &p, bool pp, int blocks, hipStream_t s) {
  if constexpr (PRO == PRO_NORM || PRO == PRO_NORM_ROPE) {
    if (p.gk) {  // mode 'full': general kernel with the per-tile K prologue
      hipLaunchKernelGGL((attn_fwd_kernel<D, BN, CAUSAL, PRO, ST, true>), dim3(blocks), dim3(256), 0, s, p);
      launch_log_add(reinterpret_cast<const void *>(&attn_fwd_kernel<D, BN, CAUSAL, PRO, ST, true>),
                     fwd_name<D, BN, CAUSAL, PRO, ST, true>(), blocks, 256);
      return hipGetLastError();
    }
  }
  if constexpr (D == 128) {
    if (pp) {
      if (p.vt) {
        hipLaunchKernelGGL((attn_pp_kernel<CAUSAL, PRO, ST, true>), dim3(blocks), dim3(512), 0, s, p);
        launch_log_add(reinterpret_cast<const void *>(&attn_pp_kernel<CAUSAL, PRO, ST, true>),
                       pp_name<CAUSAL, PRO, ST, true>(), blocks, 512);
      } else {
        hipLaunchKernelGGL((attn_pp_kernel<CAUSAL, PRO, ST, false>), dim3(blocks), dim3(512), 0, s, p);
        launch_log_add(reinterpret_cast<const void *>(&attn_pp_kernel<CAUSAL, PRO, ST, false>),
                       pp_name<CAUSAL, PRO, ST, false>(), blocks, 512);
      }
      return hipGetLastError();
    }
  }
  hipLaunchKernelGGL((attn_fwd_kernel<D, BN, CAUSAL, PRO, ST>), dim3(blocks), dim3(256), 0, s, p);
  launch_log_add(reinterpret_cast<const void *>(&attn_fwd_kernel<D, BN, CAUSAL, PRO, ST, false>),
                 fwd_name<D, BN, CAUSAL, PRO, ST, false>(), blocks, 256);
  return hipGetLastError();
}

template <int D, int BN, bool CAUSAL>
hipError_t dispatch_pro(const AttnParams &p, int pro, int st, bool pp, int blocks, hipStream_t s) {
  switch (pro) {
    case PRO_NONE: return launch_t<D, BN, CAUSAL, PRO_NONE, ST_FP32>(p, pp, blocks, s);
    case PRO_FACTORED_READ: return launch_t<D, BN, CAUSAL, PRO_FACTORED_READ, ST_FP32>(p, pp, blocks, s);
    case PRO_FACTORED_CALC: return launch_t<D, BN, CAUSAL, PRO_FACTORED_CALC, ST_FP32>(p, pp, blocks, s);
    case PRO_NORM:
      if (st == ST_HF) return launch_t<D, BN, CAUSAL, PRO_NORM, ST_HF>(p, pp, blocks, s);
      if (st == ST_LEGACY) return launch_t<D, BN, CAUSAL, PRO_NORM, ST_LEGACY>(p, pp, blocks, s);
      return launch_t<D, BN, CAUSAL, PRO_NORM, ST_FP32>(p, pp, blocks, s);
    case PRO_NORM_ROPE:
      if (st == ST_HF) return launch_t<D, BN, CAUSAL, PRO_NORM_ROPE, ST_HF>(p, pp, blocks, s);
      if (st == ST_LEGACY) return launch_t<D, BN, CAUSAL, PRO_NORM_ROPE, ST_LEGACY>(p, pp, blocks, s);
      return launch_t<D, BN, CAUSAL, PRO_NORM_ROPE, ST_FP32>(p, pp, blocks, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace

// The ping-pong kernel needs D = 128 and an even GQA ratio, and pays off from
// 24 query blocks of 128 rows (S > 2944): below that, 2-4 tile rounds per
// CU leave its 8-wave workgroups unbalanced and the general kernel (two
// 4-wave workgroups per CU) is faster (measured on MI355X: S=2048 causal
// 50.8 vs 56.9 us, B=4 S=1000 53.1 vs 56.8 us; S=4096 145 vs 134 us).
bool attention_uses_pp(int64_t Hq, int64_t Hkv, int64_t S, int64_t D) {
  constexpr int64_t PP_MIN_QBLOCKS = 24;
  return D == 128 && (Hq / Hkv) % 2 == 0 && (S + 127) / 128 >= PP_MIN_QBLOCKS;
}

namespace {

// Compute units of the current device (256 on MI355X), cached per device;
// 256 when no device can be queried.  Scheduling only: results never depend
// on it.
int64_t device_cus() {
  static std::atomic<int> cached[64];  // 0: not queried yet (host threads may race; every writer stores the same value)
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int v = cached[dev].load(std::memory_order_relaxed);
  if (v == 0) {
    int n = 0;
    v = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0 ? n : 256;
    cached[dev].store(v, std::memory_order_relaxed);
  }
  return v;
}

// Split-KV plan for the general kernel at D = 256, which runs one workgroup
// per CU: with no more work items than CUs, longest-first ordering cannot
// balance a causal grid (the heaviest query block alone sets the time, and
// no co-resident workgroup fills the gap).  Blocks with more key tiles than
// half the maximum are then split into two halves of their key range (the
// second holds the diagonal), and all items are listed longest first.  At
// D = 128 two workgroups share each CU and one already keeps it nearly
// busy, so the extra prologues of a split cost more than the balance gains.

// Workspace layout: a counter region of the same size for every shape (one
// 4-byte arrival counter per split (block, head) pair, at most
// SPLIT_MAX_PAIRS; a plan has at most B*Hq*nqb <= CUs pairs), then the
// partial results.  Because no shape's partials ever land in the counter
// region and every launch leaves the counters it used at zero, a workspace
// zero-filled once stays valid for any sequence of shapes launched on it.
constexpr int64_t SPLIT_MAX_PAIRS = 1024;
constexpr int64_t SPLIT_COUNTER_BYTES = SPLIT_MAX_PAIRS * 4;

struct SplitPlan {
  int n_items = 0, n_split = 0;
  int16_t qb[MAX_SPLIT_ITEMS], t0[MAX_SPLIT_ITEMS], t1[MAX_SPLIT_ITEMS], sid[MAX_SPLIT_ITEMS];
};

bool plan_split(int64_t B, int64_t Hq, int64_t S, int64_t D, bool causal, int64_t cus, SplitPlan &pl) {
  const int64_t BM = 128, BN = D == 128 ? 64 : 32;
  const int64_t nqb = (S + BM - 1) / BM;
  if (D != 256 || !causal || nqb < 2 || B * Hq * nqb > cus) return false;
  auto tiles = [&](int64_t qb) { return ((qb + 1) * BM < S ? (qb + 1) * BM : S) + BN - 1; };
  const int64_t t_max = tiles(nqb - 1) / BN;
  const int64_t half = (t_max + 1) / 2;
  struct Item { int qb, t0, t1, sid; };
  Item items[MAX_SPLIT_ITEMS];
  int n = 0, n_split = 0;
  for (int64_t qb = 0; qb < nqb; ++qb) {
    const int nt = (int)(tiles(qb) / BN);
    if (nt > half) {
      if (n + 2 > MAX_SPLIT_ITEMS) return false;
      const int mid = (nt + 1) / 2;
      items[n++] = {(int)qb, 0, mid, n_split};
      items[n++] = {(int)qb, mid, nt, n_split};
      ++n_split;
    } else {
      if (n + 1 > MAX_SPLIT_ITEMS) return false;
      items[n++] = {(int)qb, 0, nt, -1};
    }
  }
  if (n_split == 0 || n_split * B * Hq > SPLIT_MAX_PAIRS) return false;
  // longest first (insertion sort: n <= 128)
  for (int i = 1; i < n; ++i)
    for (int j = i; j > 0 && items[j].t1 - items[j].t0 > items[j - 1].t1 - items[j - 1].t0; --j) {
      const Item t = items[j]; items[j] = items[j - 1]; items[j - 1] = t;
    }
  pl.n_items = n;
  pl.n_split = n_split;
  for (int i = 0; i < n; ++i) {
    pl.qb[i] = (int16_t)items[i].qb; pl.t0[i] = (int16_t)items[i].t0;
    pl.t1[i] = (int16_t)items[i].t1; pl.sid[i] = (int16_t)items[i].sid;
  }
  return true;
}

int64_t split_partial_bytes(int64_t pairs, int64_t D) { return pairs * 2 * (D / 2 + 2) * 256 * 4; }

}  // namespace

int64_t attention_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t D, bool causal) {
  if (attention_uses_pp(Hq, Hkv, S, D)) return 0;
  SplitPlan pl;
  if (!plan_split(B, Hq, S, D, causal, device_cus(), pl)) return 0;
  const int64_t pairs = (int64_t)pl.n_split * B * Hq;
  return SPLIT_COUNTER_BYTES + split_partial_bytes(pairs, D);
}

int64_t attention_workspace_counter_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t D, bool causal) {
  if (attention_uses_pp(Hq, Hkv, S, D)) return 0;
  SplitPlan pl;
  if (!plan_split(B, Hq, S, D, causal, device_cus(), pl)) return 0;
  return SPLIT_COUNTER_BYTES;
}

hipError_t launch_attention(const AttnArgs &a, hipStream_t stream) {
  constexpr double LOG2E = 1.4426950408889634;
  AttnParams p;
  p.n_items = 0;
  p.pp_units = 0;
  p.pp_hpg = 1;
  p.slot2 = 0;
  p.counters = nullptr;
  p.partials = nullptr;
  p.q = a.q; p.k = a.k; p.v = a.v; p.gq = a.gq; p.cos = a.cos; p.sin = a.sin;
  p.gk = a.gk;
  p.out = a.out; p.inv = a.inv;
  p.vt = nullptr;
  p.S = a.S;
  p.B = (int)a.B; p.Hq = (int)a.Hq; p.Hkv = (int)a.Hkv;
  p.eps = a.eps;
  const bool factored = a.prologue == PRO_FACTORED_READ || a.prologue == PRO_FACTORED_CALC;
  // rope:636 SCALE*log2e; qk:621 D**-.5*log2e (both formed in double, then FP32)
  p.c_scale = (float)((factored ? 1.0 / sqrt((double)a.D) : a.scale) * LOG2E);
  const int BM = 128;
  p.n_qblocks = (int)((a.S + BM - 1) / BM);
  const int G = p.Hq / p.Hkv;
  const bool pp = attention_uses_pp(a.Hq, a.Hkv, a.S, a.D) && a.gk == nullptr;  // mode 'full': general kernel
  if (pp && a.vt && a.S % 8 == 0) p.vt = a.vt;  // V^T rows must be 16-byte aligned
  int blocks;
  if (pp) {
    p.pp_hpg = G % 4 == 0 ? 2 : 1;
    p.n_qblocks = (int)((a.S + BM / p.pp_hpg - 1) / (BM / p.pp_hpg));
    const int npairs = p.B * p.Hkv * (G / (2 * p.pp_hpg));
    p.xcd_remap = ((p.B * p.Hkv) % 8 == 0 && npairs % 8 == 0) ? 1 : 0;
    blocks = p.n_qblocks * npairs;
    // persistent mode when the (long, short) pairs fill every CU equally
    const int64_t cus = device_cus();
    const int64_t units = (int64_t)npairs * ((p.n_qblocks + 1) / 2);
    if (a.causal && p.xcd_remap && cus % 8 == 0 && units % cus == 0) {
      p.pp_units = (int)units;
      blocks = (int)cus;
    }
  } else {
    const int nbh = p.B * p.Hq;
    p.xcd_remap = (nbh % 8 == 0 && (p.B * p.Hkv) % 8 == 0) ? 1 : 0;
    blocks = p.n_qblocks * nbh;
    SplitPlan pl;
    if (a.work && plan_split(a.B, a.Hq, a.S, a.D, a.causal, device_cus(), pl)) {
      const int64_t pairs = (int64_t)pl.n_split * nbh;
      if (a.work_bytes >= SPLIT_COUNTER_BYTES + split_partial_bytes(pairs, a.D)) {
        p.n_items = pl.n_items;
        for (int i = 0; i < pl.n_items; ++i) {
          p.it_qb[i] = pl.qb[i]; p.it_t0[i] = pl.t0[i]; p.it_t1[i] = pl.t1[i]; p.it_sid[i] = pl.sid[i];
        }
        p.counters = (int *)a.work;
        p.partials = (float *)((char *)a.work + SPLIT_COUNTER_BYTES);
        blocks = pl.n_items * nbh;
      }
    }
    // D = 128, causal, all workgroups resident in one round of two per CU:
    // pair each CU's long block with a short one (the head stays the same,
    // as bid and bid + cus map to the same head when cus % nbh == 0)
    const int64_t cus = device_cus();
    if (a.causal && a.D == 128 && p.n_items == 0 && cus % nbh == 0 && blocks > cus && blocks <= 2 * cus)
      p.slot2 = (int)cus;
  }
  if (a.D == 128) {
    return a.causal ? dispatch_pro<128, 64, true>(p, a.prologue, a.style, pp, blocks, stream)
                    : dispatch_pro<128, 64, false>(p, a.prologue, a.style, pp, blocks, stream);
  }
  return a.causal ? dispatch_pro<256, 32, true>(p, a.prologue, a.style, false, blocks, stream)
                  : dispatch_pro<256, 32, false>(p, a.prologue, a.style, false, blocks, stream);
}

}  // namespace kfmi
