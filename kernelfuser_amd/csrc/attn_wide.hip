// Wide-wave attention kernel (attn_ww_kernel) and its launcher; shared
// device code in attn_common.h.
#include <cstdio>
#include <string>
#include <type_traits>

#include "attn_common.h"

namespace kfmi {
namespace {

// ---------------------------------------------------------------------------
// Wide-wave kernel: D=128, BN=64, GQA ratio a multiple of 4.  One workgroup =
// 4 waves, one per SIMD.  A work item is the four Q heads of one GQA group x
// 64 query rows; wave w holds all 64 rows of head w of the group as two
// 32-row sets (j = 0: rows q0 + lr, j = 1: rows q0 + 32 + lr).  Each staged
// K/V tile therefore serves 256 query rows, and every K or V operand read
// from LDS feeds two MFMAs, one per row set.  The wave pipelines its own tile
// loop: iteration t issues GEMM1 of tile t+1 and GEMM2 of tile t as one
// stream of 64 MFMAs, and computes the probabilities of tile t (exp2, BF16
// packing, row sums) between them, one 16-key step ahead of the GEMM2 MFMAs
// that consume them.  One barrier per tile; K and V double-buffered.
//
// Softmax: lean.  The first tile of an item sets the shift (FOLD: one shift
// per lane, the larger of its two rows' maxima, carried into every later
// GEMM1 as the accumulator's start value; otherwise each row's own max);
// later tiles never rescale.  A shift is exact for any value as long as no
// probability, row sum or output accumulator overflows; the sweep ends with
// a check of every row sum and accumulator, and a workgroup in which any of
// them is not finite redoes the item with the exact online softmax.
// ---------------------------------------------------------------------------

// Q prologue of a wide wave: two query rows per lane (row sets j = 0, 1),
// each into GEMM1 B operands exactly as q_prologue does for one row, with the
// same rounding points per style.  Every load of both rows is issued before
// the first wait.  Staged table rows (PRO_NORM_ROPE): the lane's chunk 2c+g of
// row set j is at tcos/tsin + j*32*2D + off[c]; the wait for the staging
// copies and the barrier happen inside.
template <int D, int PRO, int ST, bool FOLD>
__device__ __forceinline__ void q_prologue_ww(const AttnParams &p, int64_t qoff, const int (&qrow)[2], int g,
                                              bf16x8_t (&qreg)[2][D / 16], float (&cl)[2],
                                              const unsigned char *tcos, const unsigned char *tsin,
                                              const uint32_t (&off)[8]) {
  constexpr int NC = D / 16, HC = NC / 2;
  const uint16_t *qbase = p.q + qoff * D;
  const u32x4_t zero = {0u, 0u, 0u, 0u};
  u32x4_t raw[2][NC];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const bool qvalid = qrow[j] < p.S;
#pragma unroll
    for (int c = 0; c < NC; ++c) raw[j][c] = qvalid ? ld16(qbase + (int64_t)qrow[j] * D + 16 * c + 8 * g) : zero;
    cl[j] = p.c_scale;
  }
  if constexpr (PRO == PRO_NONE) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int c = 0; c < NC; ++c) qreg[j][c] = as_bf16x8(raw[j][c]);
  } else if constexpr (PRO == PRO_FACTORED_READ) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
      for (int c = 0; c < NC; ++c) qreg[j][c] = as_bf16x8(raw[j][c]);
      cl[j] = (qrow[j] < p.S ? p.inv[qoff + qrow[j]] : 1.0f) * p.c_scale;  // qk:621
    }
  } else {
    constexpr bool TAB = PRO == PRO_NORM_ROPE;
    constexpr bool GAM = PRO == PRO_NORM || PRO == PRO_NORM_ROPE;
    u32x4_t graw[GAM ? NC : 1];
    if constexpr (GAM) {
#pragma unroll
      for (int c = 0; c < NC; ++c) graw[c] = ld16(p.gq + 16 * c + 8 * g);
    }
    float inv[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      float ss = 0.f;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        float x[8];
        unpack8(raw[j][c], x);
#pragma unroll
        for (int e = 0; e < 8; ++e) ss = __fmaf_rn(x[e], x[e], ss);
      }
      ss = sum_halves(ss);
      inv[j] = rsqrt_rn(ss * (1.0f / D) + p.eps);
    }
    u32x4_t craw[TAB ? 2 : 1][TAB ? NC : 1], sraw[TAB ? 2 : 1][TAB ? NC : 1];
    if constexpr (TAB) {
      wait_copies();
      __syncthreads();
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          craw[j][c] = *reinterpret_cast<const u32x4_t *>(tcos + j * 32 * 2 * D + off[c]);
          sraw[j][c] = *reinterpret_cast<const u32x4_t *>(tsin + j * 32 * 2 * D + off[c]);
        }
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      if constexpr (PRO == PRO_FACTORED_CALC) {
#pragma unroll
        for (int c = 0; c < NC; ++c) qreg[j][c] = as_bf16x8(raw[j][c]);
        if (p.inv != nullptr && g == 0 && qrow[j] < p.S) p.inv[qoff + qrow[j]] = inv[j];  // qk:597-601
        cl[j] = inv[j] * p.c_scale;                                                       // qk:621
      } else {
#pragma unroll
        for (int c = 0; c < HC; ++c) {
          const int c2 = c + HC;
          float x1[8], x2[8], g1[8], g2[8], n1[8], n2[8], y1[8], y2[8];
          unpack8(raw[j][c], x1);
          unpack8(raw[j][c2], x2);
          unpack8(graw[c], g1);
          unpack8(graw[c2], g2);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            n1[e] = norm_elem<ST>(x1[e], inv[j], g1[e]);
            n2[e] = norm_elem<ST>(x2[e], inv[j], g2[e]);
          }
          if constexpr (TAB) {
            float cs1[8], sn1[8], cs2[8], sn2[8];
            unpack8(craw[j][c], cs1);
            unpack8(sraw[j][c], sn1);
            unpack8(craw[j][c2], cs2);
            unpack8(sraw[j][c2], sn2);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              y1[e] = rope_elem<ST>(n1[e], n2[e], cs1[e], sn1[e], true);
              y2[e] = rope_elem<ST>(n2[e], n1[e], cs2[e], sn2[e], false);
            }
          } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) { y1[e] = n1[e]; y2[e] = n2[e]; }
          }
          if constexpr (FOLD) {
#pragma unroll
            for (int e = 0; e < 8; ++e) { y1[e] = __fmul_rn(y1[e], p.c_scale); y2[e] = __fmul_rn(y2[e], p.c_scale); }
          }
          qreg[j][c] = as_bf16x8(pack8(y1));
          qreg[j][c2] = as_bf16x8(pack8(y2));
        }
        if constexpr (FOLD) cl[j] = 1.0f;
      }
    }
  }
}

// Masks of one key tile for both row sets (keys past the row (causal) or past
// S); register i of block kb holds key kt + 32*kb + 8*(i/4) + 4*g + i%4.
// Blocks kb < NKB, registers i < NI only (the first key step: 1, 8).
template <bool CAUSAL, int NKB, int NI>
__device__ __forceinline__ void ww_mask(f32x16_t (&s)[2][2], int kt, int q0, int lr, int64_t S, int g) {
  const int last = (int)(S - 1);
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int qrow = q0 + 32 * j + lr;
    const int lim = (CAUSAL ? (qrow < last ? qrow : last) : last) - kt - 4 * g;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int i = 0; i < NI; ++i)
        if (32 * kb + 8 * (i >> 2) + (i & 3) > lim) s[j][kb][i] = -INFINITY;
  }
}

// v_mfma_f32_32x32x16_bf16 as inline assembly, so that each operand sits in
// the register file this kernel needs: scores in VGPRs (the VALU reads them),
// O and the Q operands in AGPRs.  (With the builtin the compiler puts every
// accumulator of a kernel in one file, and O plus two score buffers do not
// fit in the 256 AGPRs.)  The compiler does not know these are MFMAs, so the
// kernel keeps their dependency distances itself.  For this MFMA on gfx950
// the compiler's own hazard rules are: none for an accumulation chain on one
// register, 2 wait states from a VALU write to an MFMA operand read, 12 from
// an MFMA result to any other instruction that reads it (and an MFMA source
// register may be overwritten right after issue).  The loop below consumes
// every MFMA result, and feeds every VALU result to an MFMA, at least eight
// MFMAs later; everywhere else an explicit wait (mfma_settle, s_nop) pads the
// gap, on operands that tie the waiting to the registers concerned.
__device__ __forceinline__ void mfma_v(f32x16_t &d, const bf16x8_t &a, const bf16x8_t &b) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(d) : "v"(a), "a"(b));
}
__device__ __forceinline__ void mfma_v_from(f32x16_t &d, const bf16x8_t &a, const bf16x8_t &b, const f32x16_t &c) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %3" : "=&v"(d) : "v"(a), "a"(b), "v"(c));
}
__device__ __forceinline__ void mfma_v_zero(f32x16_t &d, const bf16x8_t &a, const bf16x8_t &b) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(d) : "v"(a), "a"(b));
}
__device__ __forceinline__ void mfma_a(f32x16_t &d, const bf16x8_t &a, const bf16x8_t &b) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(d) : "v"(a), "v"(b));
}
// 16 wait states after the last MFMA writing these registers, before any
// other instruction reads them.
__device__ __forceinline__ void mfma_settle(f32x16_t (&s)[2][2]) {
  asm volatile("s_nop 7\n\ts_nop 7" : "+v"(s[0][0]), "+v"(s[0][1]), "+v"(s[1][0]), "+v"(s[1][1]));
}
__device__ __forceinline__ void mfma_settle_acc(f32x16_t (&o)[2][4]) {
  asm volatile("s_nop 7\n\ts_nop 7"
               : "+a"(o[0][0]), "+a"(o[0][1]), "+a"(o[0][2]), "+a"(o[0][3]), "+a"(o[1][0]), "+a"(o[1][1]),
                 "+a"(o[1][2]), "+a"(o[1][3]));
}
// Pins values into AGPRs (the copies the compiler makes land before this
// point), then 2 wait states so that an MFMA may read them next.
__device__ __forceinline__ void pin_acc(f32x16_t (&o)[2][4]) {
  asm volatile("s_nop 1"
               : "+a"(o[0][0]), "+a"(o[0][1]), "+a"(o[0][2]), "+a"(o[0][3]), "+a"(o[1][0]), "+a"(o[1][1]),
                 "+a"(o[1][2]), "+a"(o[1][3]));
}
__device__ __forceinline__ void pin_q(bf16x8_t (&q)[2][8]) {
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int c = 0; c < 8; ++c) asm volatile("" : "+a"(q[j][c]));
  asm volatile("s_nop 1");
}
// 2 wait states after VALU writes of these MFMA operands.
__device__ __forceinline__ void valu_settle(bf16x8_t (&pb)[2]) { asm volatile("s_nop 1" : "+v"(pb[0]), "+v"(pb[1])); }
__device__ __forceinline__ void valu_settle(f32x16_t &c) { asm volatile("s_nop 1" : "+v"(c)); }
__device__ __forceinline__ void valu_settle(bf16x8_t (&px)[2][4]) {
  asm volatile("s_nop 1"
               : "+v"(px[0][0]), "+v"(px[0][1]), "+v"(px[0][2]), "+v"(px[0][3]), "+v"(px[1][0]), "+v"(px[1][1]),
                 "+v"(px[1][2]), "+v"(px[1][3]));
}

template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F &&f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

template <bool CAUSAL, int PRO, int ST>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void attn_ww_kernel(AttnParams p) {
  constexpr int D = 128, BN = 64, RB = 2 * D, BMI = 64;
  constexpr int TILE = BN * RB;         // 16 KiB
  constexpr int LPW = TILE / 1024 / 4;  // copies per wave per tile (4)
  constexpr int NC = D / 16, NDB = D / 32;
  constexpr int K0 = 0, K1 = TILE, V0 = 2 * TILE, V1 = 3 * TILE;
  // Rotary-table rows of the item's 64 positions, shared by its four heads.
  constexpr int TAB = 4 * TILE, TAB_BYTES = BMI * RB;
  constexpr bool STAGE_TAB = PRO == PRO_NORM_ROPE;
  constexpr bool FOLD = ST == ST_FP32 && (PRO == PRO_NORM || PRO == PRO_NORM_ROPE);

  __shared__ __attribute__((aligned(1024))) unsigned char smem[4 * TILE + (STAGE_TAB ? 2 * TAB_BYTES : 0)];

  clock_stamp<false>(p.stamps);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // the wave's head within the item
  const int g = lane >> 5, lr = lane & 31;
  const int64_t S = p.S;
  const int G = p.Hq / p.Hkv;
  const int HP = G / 4;  // items of one query block per KV head
  const int npairs = p.B * p.Hkv * HP;
  const uint32_t lds0 = (uint32_t)reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) unsigned char *)smem);

  auto run = [&](const int qb, const int kvi, const int jq) {
  const int b = kvi / p.Hkv;
  const int kvh = kvi - b * p.Hkv;
  const int h = kvh * G + 4 * jq + w;
  const int64_t qoff = ((int64_t)b * p.Hq + h) * S;
  const int64_t kvoff = ((int64_t)b * p.Hkv + kvh) * S;
  const uint32_t head_bytes = (uint32_t)(S * RB);
  const i32x4_t krs = buffer_rsrc(p.k + kvoff * D, head_bytes);
  const i32x4_t vrs = buffer_rsrc(p.v + kvoff * D, head_bytes);
  uint32_t kvo[LPW], vvo[LPW];
#pragma unroll
  for (int i = 0; i < LPW; ++i) {
    kvo[i] = copy_lane_offset<D>(w * LPW + i, lane, false);
    vvo[i] = copy_lane_offset<D>(w * LPW + i, lane, true);
  }
  auto copy_k = [&](int t, int buf) {
#pragma unroll
    for (int i = 0; i < LPW; ++i) copy16_to_lds(krs, lds0 + buf + (w * LPW + i) * 1024, kvo[i] + (uint32_t)(t * TILE));
  };
  auto copy_v = [&](int t, int buf) {
#pragma unroll
    for (int i = 0; i < LPW; ++i) copy16_to_lds(vrs, lds0 + buf + (w * LPW + i) * 1024, vvo[i] + (uint32_t)(t * TILE));
  };

  const int q0 = qb * BMI;
  const int qrow[2] = {q0 + lr, q0 + 32 + lr};
  const int64_t kv_end = CAUSAL ? ((int64_t)(qb + 1) * BMI < S ? (int64_t)(qb + 1) * BMI : S) : S;
  const int nT = (int)((kv_end + BN - 1) / BN);
  // a tile needs masks when it reaches past the wave's first row (causal) or past S
  auto need_mask = [&](int t) { return (CAUSAL && t * BN + BN - 1 > q0) || ((int64_t)t * BN + BN > S); };

  uint32_t kra[8], vra[4];
  lds_read_offsets<D>(lane, kra, vra);

  copy_k(0, K0);
  if constexpr (STAGE_TAB) {
    // 16 copies of 4 rows per table, 4 per wave, with the K tiles' chunk
    // swizzle (kra[c] then addresses the lane's row chunk)
    const i32x4_t crs = buffer_rsrc(p.cos, head_bytes);
    const i32x4_t srs = buffer_rsrc(p.sin, head_bytes);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = 4 * w + i;
      const uint32_t voff = copy_lane_offset<D>(j, lane, false) + (uint32_t)(q0 * RB);
      copy16_to_lds(crs, lds0 + TAB + j * 1024, voff);
      copy16_to_lds(srs, lds0 + TAB + TAB_BYTES + j * 1024, voff);
    }
  }
  if (nT > 1) copy_k(1, K1);
  copy_v(0, V0);

  bf16x8_t qreg[2][NC];
  float cl[2];
  q_prologue_ww<D, PRO, ST, FOLD>(p, qoff, qrow, g, qreg, cl, smem + TAB, smem + TAB + TAB_BYTES, kra);
  if constexpr (!STAGE_TAB) {
    wait_copies();
    __syncthreads();
  }
  f32x16_t o[2][NDB];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int db = 0; db < NDB; ++db) o[j][db] = f32x16_t{};
  pin_acc(o);
  pin_q(qreg);

  float lp[2][2] = {{0.f, 0.f}, {0.f, 0.f}};  // [row set][partial] row sums
  float nm[2] = {0.f, 0.f};                   // !FOLD: minus each row's shift
  f32x16_t cinit;                             // FOLD: GEMM1 start value, minus the lane's shift

  // K operand of chunk c of GEMM1 part R (key block R/2, chunk 4*(R%2) + c);
  // one half of the V operand of key step R, d block db.
  auto kread = [&](int buf, auto rr, auto cc) {
    constexpr int R = decltype(rr)::value, C = decltype(cc)::value;
    return *reinterpret_cast<const bf16x8_t *>(smem + buf + (R / 2) * 32 * RB + kra[4 * (R % 2) + C]);
  };
  auto vread = [&](int buf, auto rr, auto dd, auto hh) {
    constexpr int R = decltype(rr)::value, DB = decltype(dd)::value, HH = decltype(hh)::value;
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t *)(smem + buf + 16 * R * RB + vra[DB] + HH * 8 * RB));
  };
  auto vop = [](const i16x4_t &lo, const i16x4_t &hi) {
    return __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  };

  // Probabilities of one 16-key step R of the scores s (registers
  // 8*(R%2) .. of block R/2, keys 16R + 8*(e/4) + 4g + e%4: the order of the
  // GEMM2 operands) -> P^T operands out[j], and the BF16-rounded values (the
  // ones the MFMA multiplies) into the row sums through v_dot2 with (1, 1).
  // FOLD: scores are logit - shift.  Three kinds of operations, on element
  // m = 8j + e (of 16) and pair p = 4j + i (of 8): exp2 of an element, the
  // BF16 pack of a pair, the row-sum update of a pair.
  float pe[2][8];
  uint32_t pw[2][4];  // a plain array: a bit cast of an element of a vector-typed array read the wrong element
  uint32_t one_bits = 0x3f803f80u;  // BF16 (1, 1), kept in a register rather than as a literal
  asm volatile("" : "+v"(one_bits));
  auto exp_op = [&](auto mm, auto rr, const f32x16_t (&s)[2][2]) {
    constexpr int M = decltype(mm)::value, R = decltype(rr)::value;
    constexpr int J = M / 8, E = M % 8, KB = R / 2, H = 8 * (R % 2) + E;
    pe[J][E] = __builtin_amdgcn_exp2f(FOLD ? s[J][KB][H] : __builtin_fmaf(s[J][KB][H], cl[J], nm[J]));
  };
  auto pack_op = [&](auto pp, bf16x8_t (&out)[2]) {
    constexpr int P = decltype(pp)::value, J = P / 4, I = P % 4;
    pw[J][I] = pack_bf16x2(pe[J][2 * I], pe[J][2 * I + 1]);
    if constexpr (I == 3) {
      const u32x4_t v = {pw[J][0], pw[J][1], pw[J][2], pw[J][3]};
      out[J] = __builtin_bit_cast(bf16x8_t, v);
    }
  };
  auto sum_op = [&](auto pp) {
    constexpr int P = decltype(pp)::value, J = P / 4, I = P % 4;
    lp[J][I & 1] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, pw[J][I]),
                                                   __builtin_bit_cast(bf16x2_t, one_bits), lp[J][I & 1], false);
  };
  // VALU work of slot m of a 16-slot round, skewed so that no operation
  // waits for the one before it: the exp2 of element m; at even slots from
  // 4 the pack of pair m/2 - 2, at odd slots from 7 the row sum of pair
  // (m-7)/2; the pairs left over (packs of 6, 7; sums of 5, 6, 7) are done
  // in slots 0-5 of the next round (TAIL), on the previous step's values
  // (out_prev: its P^T operands, completed at slot 2).
  auto valu_slot = [&](auto mm, auto rr, auto tail, const f32x16_t (&s)[2][2], bf16x8_t (&out)[2],
                       bf16x8_t (&out_prev)[2]) {
    constexpr int M = decltype(mm)::value;
    constexpr bool TAIL = decltype(tail)::value;
    if constexpr (TAIL && M == 0) pack_op(std::integral_constant<int, 6>{}, out_prev);
    if constexpr (TAIL && M == 2) pack_op(std::integral_constant<int, 7>{}, out_prev);
    if constexpr (TAIL && M % 2 == 1 && M <= 5) sum_op(std::integral_constant<int, 5 + M / 2>{});
    exp_op(mm, rr, s);
    if constexpr (M % 2 == 0 && M >= 4) pack_op(std::integral_constant<int, M / 2 - 2>{}, out);
    if constexpr (M % 2 == 1 && M >= 7) sum_op(std::integral_constant<int, (M - 7) / 2>{});
  };
  // Keeps every value of the probability pipeline where it is (an empty asm
  // that rewrites them): no later pass may sink their computation past a
  // branch that follows.
  auto pin_valu = [&](bf16x8_t (&x)[2], bf16x8_t (&y)[2]) {
    asm volatile("" : "+v"(pe[0][0]), "+v"(pe[0][1]), "+v"(pe[0][2]), "+v"(pe[0][3]), "+v"(pe[0][4]), "+v"(pe[0][5]),
                 "+v"(pe[0][6]), "+v"(pe[0][7]), "+v"(pe[1][0]), "+v"(pe[1][1]), "+v"(pe[1][2]), "+v"(pe[1][3]),
                 "+v"(pe[1][4]), "+v"(pe[1][5]), "+v"(pe[1][6]), "+v"(pe[1][7]));
    asm volatile("" : "+v"(pw[0][0]), "+v"(pw[0][1]), "+v"(pw[0][2]), "+v"(pw[0][3]), "+v"(pw[1][0]), "+v"(pw[1][1]),
                 "+v"(pw[1][2]), "+v"(pw[1][3]), "+v"(lp[0][0]), "+v"(lp[0][1]), "+v"(lp[1][0]), "+v"(lp[1][1]),
                 "+v"(x[0]), "+v"(x[1]), "+v"(y[0]), "+v"(y[1]));
  };

  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;

  f32x16_t sa[2][2], sb[2][2];
  bf16x8_t pb[2], pn[2];
  bf16x8_t kop[4];  // K operands of the current GEMM1 part

  // Round R of an iteration (tile t+1 exists): 16 MFMA slots.
  //   slots 0-7 : GEMM1 part R of tile t+1 into nxt (chunk 4*(R%2) + m/2,
  //               row set m%2); reads of V(t) step R, d block m/2, half m%2;
  //   slots 8-15: GEMM2 step R (d block (m-8)/2, row set m%2) with pbc; K
  //               reads of the next part (chunk (m-8)/2 on even m), from
  //               kbuf_next for part 0 of the next iteration.
  // Every slot also issues its share of the VALU work: probabilities of step
  // R+1 of cur (R < 3), or of step 0 of nxt (R == 3) into pout.
  // SYNC runs between slots 7 and 8 of round 3 (the tile's barrier).
  auto round = [&](auto rr, int kbuf, int vbuf, int kbuf_next, const f32x16_t (&cur)[2][2], f32x16_t (&nxt)[2][2],
                   bf16x8_t (&pbc)[2], bf16x8_t (&pout)[2], auto sync) {
    constexpr int R = decltype(rr)::value;
    i16x4_t vlo[4], vhi[4];
    bf16x8_t knext[4];
    static_for<0, 16>([&](auto mm) {
      constexpr int m = decltype(mm)::value;
      if constexpr (m < 8) {
        constexpr int c = 4 * (R % 2) + m / 2, j = m % 2, KB = R / 2;
        if constexpr (c == 0) mfma_v_from(nxt[j][KB], kop[m / 2], qreg[j][c], cinit);
        else mfma_v(nxt[j][KB], kop[m / 2], qreg[j][c]);
      } else {
        constexpr int db = (m - 8) / 2, j = m % 2;
        mfma_a(o[j][db], vop(vlo[db], vhi[db]), pbc[j]);
      }
      if constexpr (R < 3) valu_slot(mm, std::integral_constant<int, R + 1>{}, std::true_type{}, cur, pout, pbc);
      else valu_slot(mm, I0{}, std::true_type{}, nxt, pout, pbc);
      if constexpr (m < 8) {
        if constexpr (m % 2 == 0) vlo[m / 2] = vread(vbuf, rr, std::integral_constant<int, m / 2>{}, I0{});
        else vhi[m / 2] = vread(vbuf, rr, std::integral_constant<int, m / 2>{}, I1{});
      } else if constexpr (m % 2 == 0) {
        knext[(m - 8) / 2] = kread(R == 3 ? kbuf_next : kbuf, std::integral_constant<int, (R + 1) % 4>{},
                                   std::integral_constant<int, (m - 8) / 2>{});
      }
      // Finished VALU results are pinned here (an empty asm that rewrites
      // them), so that no later pass sinks their computation past the
      // barrier's branches into the slots after it.
      if constexpr (m == 7 && R == 3) {
        pin_valu(pbc, pout);
        sync();
      }
      if constexpr (m == 15 && R >= 2) pin_valu(pbc, pout);  // branches follow rounds 2 and 3
      __builtin_amdgcn_sched_barrier(0);
    });
#pragma unroll
    for (int c = 0; c < 4; ++c) kop[c] = knext[c];
  };

  // Iteration t: GEMM1 of tile t+1 from K[(t+1)%2], GEMM2 of tile t from
  // V[t%2], the probabilities of tile t (step 0 was computed by the previous
  // iteration) and of tile t+1's step 0.  Its barrier (round 3) waits for
  // K(t+2) and V(t+1) and refills the buffers this iteration read: K(t+3)
  // into K[(t+1)%2], V(t+2) into V[t%2].  Only the last tile can need masks:
  // its first step is masked before the previous iteration computes it (that
  // key block is complete by round 2), the rest at the start of its own
  // iteration.  The last iteration has no tile t+1: its GEMM1 starts from
  // -inf, so the scores it makes of finite K rows give probabilities of
  // exactly 0 and add nothing to the row sums.  An item of one tile never
  // fills that buffer, and LDS keeps whatever earlier workgroups left there:
  // NaN or inf bits make NaN row sums, which send the item to the exact redo
  // (not_finite tests the bits through an empty asm, so no build assumption
  // removes that check).  Copying a tile into the buffer for such items
  // instead made the compiler spill more registers (S=2048 non-causal, HF
  // style: 5% slower).
  auto iter = [&](auto par, int t, f32x16_t (&cur)[2][2], f32x16_t (&nxt)[2][2]) {
    constexpr int PAR = decltype(par)::value;
    constexpr int KN = PAR ? K0 : K1, VC = PAR ? V1 : V0, KO = PAR ? K1 : K0;
    if (t + 1 == nT) {
#pragma unroll
      for (int i = 0; i < 16; ++i) cinit[i] = -INFINITY;
      valu_settle(cinit);
    }
    if (need_mask(t)) ww_mask<CAUSAL, 2, 16>(cur, t * BN, q0, lr, S, g);
    auto none = [] {};
    auto sync = [&] {
      wait_copies();
      __syncthreads();
      if (t + 3 < nT) copy_k(t + 3, KN);
      if (t + 2 < nT) copy_v(t + 2, VC);
    };
    round(I0{}, KN, VC, KO, cur, nxt, pb, pn, none);
    round(I1{}, KN, VC, KO, cur, nxt, pn, pb, none);
    round(I2{}, KN, VC, KO, cur, nxt, pb, pn, none);
    if (t + 1 < nT && need_mask(t + 1)) ww_mask<CAUSAL, 1, 8>(nxt, (t + 1) * BN, q0, lr, S, g);
    round(I3{}, KN, VC, KO, cur, nxt, pn, pb, sync);
  };

  // ---- lean sweep ----
  // Tile 0: GEMM1 from zero accumulators (K(0) in K0), reads one part ahead.
  static_for<0, 4>([&](auto cc) { kop[cc] = kread(K0, I0{}, cc); });
  static_for<0, 4>([&](auto rr) {
    constexpr int R = decltype(rr)::value, KB = R / 2;
    bf16x8_t knext[4];
    static_for<0, 8>([&](auto mm) {
      constexpr int m = decltype(mm)::value, c = 4 * (R % 2) + m / 2, j = m % 2;
      if constexpr (c == 0) mfma_v_zero(sa[j][KB], kop[m / 2], qreg[j][c]);
      else mfma_v(sa[j][KB], kop[m / 2], qreg[j][c]);
      if constexpr (R < 3 && m % 2 == 0)
        knext[m / 2] = kread(K0, std::integral_constant<int, R + 1>{}, std::integral_constant<int, m / 2>{});
      __builtin_amdgcn_sched_barrier(0);
    });
    if constexpr (R < 3) {
#pragma unroll
      for (int c = 0; c < 4; ++c) kop[c] = knext[c];
    }
  });
  // The first barrier: K(1) and V(0) have landed (the prologue waited);
  // K(0)'s buffer takes K(2), V1 takes V(1); then the first K reads of
  // iteration 0 (K(1) in K1).
  wait_copies();
  __syncthreads();
  if (nT > 2) copy_k(2, K0);
  if (nT > 1) copy_v(1, V1);
  static_for<0, 4>([&](auto cc) { kop[cc] = kread(K1, I0{}, cc); });
  mfma_settle(sa);
  if (need_mask(0)) ww_mask<CAUSAL, 2, 16>(sa, 0, q0, lr, S, g);
  {
    float mx[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      float mt[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) mt[i] = fmaxf(sa[j][0][i], sa[j][1][i]);
#pragma unroll
      for (int n = 16; n > 1; n /= 2)
#pragma unroll
        for (int i = 0; i < n / 2; ++i) mt[i] = fmaxf(mt[i], mt[i + n / 2]);
      mx[j] = mt[0];
    }
    if constexpr (FOLD) {
      const float sh = max_halves(fmaxf(mx[0], mx[1]));
#pragma unroll
      for (int i = 0; i < 16; ++i) cinit[i] = -sh;
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int i = 0; i < 16; ++i) sa[j][kb][i] -= sh;
    } else {
      cinit = f32x16_t{};
#pragma unroll
      for (int j = 0; j < 2; ++j) nm[j] = -(max_halves(mx[j]) * cl[j]);
    }
    valu_settle(cinit);
  }
  // step 0 of tile 0: the operations a round makes for its own step; its
  // leftover pairs are done by the first round of the loop
  static_for<0, 16>([&](auto mm) { valu_slot(mm, I0{}, std::false_type{}, sa, pb, pn); });
  for (int t = 0;;) {
    iter(I0{}, t, sa, sb);
    if (++t >= nT) break;
    iter(I1{}, t, sb, sa);
    if (++t >= nT) break;
  }
  mfma_settle_acc(o);

  float lrow[2] = {lp[0][0] + lp[0][1], lp[1][0] + lp[1][1]};
  // Overflow check: every row sum and every accumulator must be finite.
  bool bad = not_finite(sum_halves(lrow[0]));  // |= throughout: a short circuit's branch costs the loop registers
  bad |= not_finite(sum_halves(lrow[1]));
  bad |= any_not_finite(o[0]);
  bad |= any_not_finite(o[1]);
  if (__syncthreads_or(bad)) {
    // Exact online softmax (lazy rescale), one tile at a time.
    Softmax<D, BN, CAUSAL, FOLD> sm[2];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int db = 0; db < NDB; ++db) o[j][db] = f32x16_t{};
    pin_acc(o);
    copy_k(0, K0);
    copy_v(0, V0);
    for (int t = 0; t < nT; ++t) {
      const int par = t & 1;
      wait_copies();
      __syncthreads();
      if (t + 1 < nT) {
        copy_k(t + 1, par ? K0 : K1);
        copy_v(t + 1, par ? V0 : V1);
      }
      const unsigned char *kt = smem + (par ? K1 : K0), *vt = smem + (par ? V1 : V0);
      f32x16_t s[2][2], c0[2];
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 16; ++i) c0[j][i] = sm[j].acc_init();
      valu_settle(c0[0]);
      valu_settle(c0[1]);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const bf16x8_t a = *reinterpret_cast<const bf16x8_t *>(kt + kb * 32 * RB + kra[c]);
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            if (c == 0) mfma_v_from(s[j][kb], a, qreg[j][c], c0[j]);
            else mfma_v(s[j][kb], a, qreg[j][c]);
          }
        }
      mfma_settle(s);
      bf16x8_t px[2][4];
#pragma unroll
      for (int j = 0; j < 2; ++j) sm[j].step(s[j], t, q0 + 32 * j, qrow[j], S, g, cl[j], o[j], px[j]);
      pin_acc(o);
      valu_settle(px);
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
          const unsigned char *base = vt + 16 * r * RB + vra[db];
          const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t *)(base));
          const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t *)(base + 8 * RB));
#pragma unroll
          for (int j = 0; j < 2; ++j) mfma_a(o[j][db], vop(lo, hi), px[j][r]);
        }
      mfma_settle_acc(o);
    }
    lrow[0] = sm[0].l_run;
    lrow[1] = sm[1].l_run;
  }

  __syncthreads();  // every wave is past its last K/V read: the buffers stage the epilogue
  unsigned char *tile = smem + w * (2 * 32 * RB);
#pragma unroll
  for (int j = 0; j < 2; ++j)
    store_rows_lds<D>(tile + j * 32 * RB, p.out + qoff * D, q0 + 32 * j, S, lane, lrow[j], o[j]);
  };

  // ---- work items: as in the ping-pong kernel with four-head items.
  // Persistent (pp_units > 0, causal): unit u pairs query blocks R-1-m and m
  // of one head quad, and the grid (a multiple of 8) keeps unit u on XCD
  // u % 8, the home of its KV head.  Otherwise one item per workgroup,
  // heaviest blocks first. ----
  const int R = p.n_qblocks;
  int u = blockIdx.x, phase = 0;
  for (;;) {
    int qb, kvi, jq;
    if (p.pp_units > 0) {
      if (u >= p.pp_units) break;
      const int per_kv = HP * ((R + 1) / 2);
      const int rest = u >> 3;
      kvi = (u & 7) + 8 * (rest / per_kv);
      const int rem = rest % per_kv;
      jq = rem % HP;
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
        const int xcd = r & 7, jj = r >> 3;
        kvi = xcd + 8 * (jj / HP);
        jq = jj % HP;
      } else {
        kvi = r / HP;
        jq = r - kvi * HP;
      }
    }
    run(qb, kvi, jq);
    __syncthreads();  // the next item refills the LDS buffers
  }
  clock_stamp<true>(p.stamps);
}

template <bool CAUSAL, int PRO, int ST>
const char *ww_name() {
  static const std::string n = [] {
    char b[96];
    snprintf(b, sizeof(b), "attn_ww_kernel<%s, %d, %d>", tf(CAUSAL), PRO, ST);
    return std::string(b);
  }();
  return n.c_str();
}

template <bool CAUSAL, int PRO, int ST>
hipError_t launch_ww_t(const AttnParams &p, int blocks, hipStream_t s) {
  hipLaunchKernelGGL((attn_ww_kernel<CAUSAL, PRO, ST>), dim3(blocks), dim3(256), 0, s, p);
  launch_log_add(reinterpret_cast<const void *>(&attn_ww_kernel<CAUSAL, PRO, ST>), ww_name<CAUSAL, PRO, ST>(), blocks,
                 256);
  return hipGetLastError();
}

template <bool CAUSAL>
hipError_t launch_ww_c(const AttnParams &p, int pro, int st, int blocks, hipStream_t s) {
  switch (pro) {
    case PRO_NONE: return launch_ww_t<CAUSAL, PRO_NONE, ST_FP32>(p, blocks, s);
    case PRO_FACTORED_READ: return launch_ww_t<CAUSAL, PRO_FACTORED_READ, ST_FP32>(p, blocks, s);
    case PRO_FACTORED_CALC: return launch_ww_t<CAUSAL, PRO_FACTORED_CALC, ST_FP32>(p, blocks, s);
    case PRO_NORM:
      if (st == ST_HF) return launch_ww_t<CAUSAL, PRO_NORM, ST_HF>(p, blocks, s);
      if (st == ST_LEGACY) return launch_ww_t<CAUSAL, PRO_NORM, ST_LEGACY>(p, blocks, s);
      return launch_ww_t<CAUSAL, PRO_NORM, ST_FP32>(p, blocks, s);
    case PRO_NORM_ROPE:
      if (st == ST_HF) return launch_ww_t<CAUSAL, PRO_NORM_ROPE, ST_HF>(p, blocks, s);
      if (st == ST_LEGACY) return launch_ww_t<CAUSAL, PRO_NORM_ROPE, ST_LEGACY>(p, blocks, s);
      return launch_ww_t<CAUSAL, PRO_NORM_ROPE, ST_FP32>(p, blocks, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_wide(const AttnParams &p, bool causal, int pro, int st, int blocks, hipStream_t s) {
  return causal ? launch_ww_c<true>(p, pro, st, blocks, s) : launch_ww_c<false>(p, pro, st, blocks, s);
}

}  // namespace kfmi
