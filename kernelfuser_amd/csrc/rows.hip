// Row preparation kernels for gfx950: per-(token, head) RMSNorm * gamma with
// optional rotate-half RoPE (the reference's prepare_kernel/_rows,
// src/e1_rope_publication_v1.py:550-605) and the factored no-RoPE
// preparation (src/e1_qk_publication_v3.py:592-609).
//
// Memory-bound design:
//  * a D-wide BF16 row is D/8 lanes x 16 bytes (one 16-lane DPP row for D=128);
//    rows are taken in memory order, one 16-byte chunk per lane, so a
//    workgroup covers 256/(D/8) consecutive rows and the grid streams
//    through each tensor front to back (the same rate at every B and S);
//  * the sum of squares is reduced with DPP inside the row, the rotate-half
//    partner (column d +/- D/2) is the lane D/16 away (row_ror:8 for D=128);
//  * each lane reads its position's cos/sin chunk and the gamma chunks with
//    cached loads, and the row itself with nontemporal loads and stores;
//  * FP32 internal arithmetic; the rounding points follow the selected style.
#include <cstdio>
#include <string>

#include "kfmi_device.h"
#include "kfmi_launch.h"

namespace kfmi {
namespace {

struct RowsParams {
  const uint16_t *q, *k, *gq, *gk, *cos, *sin;
  uint16_t *qn, *kn;
  float *inv;
  const uint16_t *v;  // V, transposed into vt by the extra workgroups (VT kernels)
  uint16_t *vt;
  int64_t S;
  uint32_t s32;             // S
  uint32_t heads_q, heads_k;  // B*Hq (0 for K-only launches) and B*Hkv
  uint32_t nblk;              // workgroups per unit of heads (blocks of positions)
  int hpw;                    // heads per workgroup (the kernel instance's U)
  uint32_t row_blocks;        // workgroups of the row work; V^T tiles follow
  int vt_sblocks;           // 64-row tiles per head of V
  int64_t vt_tiles;         // B * Hkv * vt_sblocks
  float eps;
};

// V -> VT per head, one 64-row tile (rows s0..s0+63 of head bh) per
// workgroup of 256 threads.  The rows are read with coalesced 16-byte loads
// into a row-major LDS tile whose 16-byte chunks are XOR-swizzled
// (chunk ^ 4*(row % 4)), then read back with ds_read_b64_tr_b16: two
// transpose reads give a lane 8 consecutive rows of one column, i.e. 16
// contiguous bytes of a VT row, stored with one 16-byte write.  Rows past S
// load as zeros and are not stored.  Requires S % 8 == 0 (16-byte aligned VT
// rows); the host checks it.
template <int D>
__device__ __forceinline__ void transpose_tile(const uint16_t *__restrict__ v, uint16_t *__restrict__ vt, int64_t S,
                                               int64_t bh, int64_t s0) {
  constexpr int TR = 64;      // rows per tile
  constexpr int RB = 2 * D;   // bytes per row
  constexpr int CPR = D / 8;  // 16-byte chunks per row
  __shared__ __attribute__((aligned(16))) unsigned char tile[TR * RB];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5;
  const uint16_t *src = v + (bh * S + s0) * D;
  const int rows = (int)((S - s0) < TR ? (S - s0) : TR);
  const u32x4_t zero = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int i = 0; i < TR * CPR / 256; ++i) {
    const int e = tid + 256 * i;
    const int r = e / CPR, c = e % CPR;
    const u32x4_t x = r < rows ? ld16_nt(src + (int64_t)r * D + 8 * c) : zero;
    *reinterpret_cast<u32x4_t *>(tile + r * RB + ((c ^ ((r & 3) << 2)) << 4)) = x;
  }
  __syncthreads();
  // Transpose reads: the 16-lane group supplies rows (lane%16)/4 + 8g (and +4
  // for the second read) of a 16-row step and 4-column runs
  // 16*((lane/16)%2) + 4*(lane%4) of a 32-wide column block; lane l then holds
  // rows 16*c2 + 8g .. +7, in order, of column 32*db + l%32.
  const int m = (lane >> 2) & 3, hh = (lane >> 4) & 1, kk = (lane >> 1) & 1;
  const int row0 = ((lane & 15) >> 2) + 8 * g;
  constexpr int NBLK = (TR / 16) * (D / 32);
  uint16_t *dst = vt + bh * D * S;
#pragma unroll
  for (int i = 0; i < NBLK / 4; ++i) {
    const int blk = w * (NBLK / 4) + i;
    const int c2 = blk / (D / 32), db = blk % (D / 32);
    const int chunk0 = 4 * db + 2 * hh + kk;  // chunk of the lane's 8-byte run
    const unsigned char *base = tile + (16 * c2 + row0) * RB + ((chunk0 ^ (m << 2)) << 4) + (lane & 1) * 8;
    const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t *)(base));
    const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t *)(base + 4 * RB));
    const int r = 16 * c2 + 8 * g;
    if (r < rows) {
      const u32x4_t x = __builtin_bit_cast(u32x4_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
      st16(dst + (int64_t)(32 * db + (lane & 31)) * S + s0 + r, x);
    }
  }
}

// Normalised element x*inv*gamma with the rounding points of a style.
template <int ST>
__device__ __forceinline__ float norm_elem(float x, float inv, float g) {
  if (ST == ST_HF) return round_bf16(round_bf16(x * inv) * g);  // rope:560-561
  if (ST == ST_LEGACY) return round_bf16(__fmul_rn(__fmul_rn(x, inv), g));  // rope:563
  return __fmul_rn(__fmul_rn(x, inv), g);  // FP32: rope:125, rope:298
}

// rotate-half output of one element: first half n*c - np*s, second half n*c + np*s.
template <int ST>
__device__ __forceinline__ float rope_elem(float n, float np, float c, float s, bool first) {
  if (ST == ST_FP32) {  // rope:129 / rope:164-167 (fp32=True): two products, one add
    // No contraction into an FMA: both products are rounded, then the sum
    // (HIP's __fmul_rn/__fadd_rn are plain * and + that the headers let the
    // compiler contract, so the operators are written here).
#pragma clang fp contract(off)
    const float p0 = n * c, p1 = np * s;
    return first ? p0 - p1 : p0 + p1;
  }
  float p0 = round_bf16(n * c), p1 = round_bf16(np * s);  // rope:578-579
  return first ? p0 - p1 : p0 + p1;  // rounded to BF16 at the store (rope:580-581)
}

template <int LPR>
__device__ __forceinline__ float row_sum(float x) {
  x = sum16(x);
  if constexpr (LPR == 32) x += __shfl_xor(x, 16);
  return x;
}

#ifndef KFMI_ROWS_NT
#define KFMI_ROWS_NT 1
#endif
// Heads per workgroup (rows per lane) of rows_kernel: two, or four for Q+K
// launches at D = 128 where the tuning runner measured four faster:
// - every style from 2^15 to 2^17 rows: HF and legacy, whose per-row
//   arithmetic is longer, 8.2 vs 9.9 us at B = 1, S = 2048 (16-21% from 40k
//   to 82k rows, 3-5% at 123k-164k); FP32 8.56-8.68 vs 8.97-9.20 us at
//   B = 1, S = 2048 (82k rows; two tuning rows) and 12.1 vs 12.3 us at
//   S = 3072, while two heads are 1-3% faster at 160k rows and more
//   (FP32 B = 1, S = 4096: 15.2 vs 15.5 us);
// - FP32 style, also at least 2^18 rows with S <= 4096: 27.2 vs 28.1-28.4
//   us at the 170 MB shapes (B >= 4), a tie at S = 8192.
// Fewer, longer workgroups lose on small launches (below 2^15 rows), and
// the K-only preparation is faster with two.
constexpr int ROWS_HPW = 2, ROWS_HPW_BIG = 4;
constexpr int64_t ROWS_BIG = (int64_t)1 << 18, ROWS_BIG_MAX_S = 4096;
constexpr int64_t ROWS_MID_MIN = (int64_t)1 << 15, ROWS_MID_END = (int64_t)1 << 17;
__device__ __forceinline__ u32x4_t ld_row(const uint16_t *p) { return KFMI_ROWS_NT ? ld16_nt(p) : ld16(p); }
__device__ __forceinline__ void st_row(uint16_t *p, const u32x4_t &v) {
  if (KFMI_ROWS_NT) st16_nt(p, v); else st16(p, v);
}

// Normalised value held by the rotate-half partner lane (lane ^ LPR/2).
template <int LPR>
__device__ __forceinline__ float partner_f32(float x) {
  if constexpr (LPR == 16) return dpp_f32<DPP_ROW_ROR8>(x);
  else return __shfl_xor(x, LPR / 2);
}

// A workgroup of 256 threads covers 256/LPR consecutive positions of HPW
// adjacent heads (Q heads (b, h) of [B,Hq,S,D], absent for K-only launches,
// then K heads), one 16-byte chunk per lane and head.  Consecutive
// workgroups take consecutive positions of the same heads, so the rows in
// flight at any time form one contiguous region of each tensor, whatever B,
// H and S are.  A lane loads its chunk of each head's row (nontemporal) and
// its cos/sin and gamma chunks once for all HPW rows (cached loads: the
// tables and gamma are read once per HPW rows rather than once per row).
// The rotate-half partner's normalised values come from the partner lane,
// which computes exactly them for its own chunk.  Lanes past the end (a
// position >= S, or a head past the tensor's last when HPW does not divide
// its head count) load the last position / head, so every load stays in
// bounds and unconditional, and store nothing (outputs may alias inputs).
template <int D, int ST, bool ROPE, bool ONLY_K, bool VT, int U>
__global__ __launch_bounds__(256) void rows_kernel(RowsParams p) {
  constexpr int LPR = D / 8;      // lanes per row
  constexpr int RPB = 256 / LPR;  // positions per workgroup
  constexpr int HALF = LPR / 2;
  const uint32_t blk = blockIdx.x;
  if constexpr (VT) {
    // Workgroups past the row work transpose V tiles (same launch).
    if (blk >= p.row_blocks) {
      const int64_t t = (int64_t)(blk - p.row_blocks);
      if (t < p.vt_tiles) transpose_tile<D>(p.v, p.vt, p.S, t / p.vt_sblocks, (t % p.vt_sblocks) * 64);
      return;  // workgroup-uniform
    }
  }
  // Workgroup -> (unit of U heads, block of RPB positions): Q units first.
  const uint32_t heads_q = ONLY_K ? 0u : p.heads_q;
  const uint32_t units_q = (heads_q + U - 1) / U;
  const uint32_t unit = blk / p.nblk;
  const uint32_t bpos = blk - unit * p.nblk;
  const bool is_q = unit < units_q;  // workgroup-uniform
  const uint32_t nh = is_q ? heads_q : p.heads_k;
  const uint32_t h0 = (is_q ? unit : unit - units_q) * U;
  uint32_t pos = bpos * RPB + threadIdx.x / LPR;
  const bool pvalid = pos < p.s32;
  if (!pvalid) pos = p.s32 - 1;  // loads stay in bounds; nothing is stored for this lane
  const uint32_t lc = threadIdx.x % LPR;
  const bool first = lc < HALF;
  const char *src = reinterpret_cast<const char *>(is_q ? p.q : p.k);
  char *dst = reinterpret_cast<char *>(is_q ? p.qn : p.kn);
  const uint16_t *g = is_q ? p.gq : p.gk;

  uint32_t off[U];  // byte offsets of the lane's chunks (< 2^32: each tensor has < 2^31 elements)
  uint32_t row[U];
  u32x4_t xv[U];
#pragma unroll
  for (int i = 0; i < U; ++i) {
    const uint32_t hh = min(h0 + i, nh - 1);
    row[i] = hh * p.s32 + pos;
    off[i] = row[i] * (uint32_t)(2 * D) + lc * 16u;
    xv[i] = ld_row(reinterpret_cast<const uint16_t *>(src + off[i]));
  }
  const u32x4_t g_own = ld16(g + lc * 8);
  u32x4_t cv, sv, gqv;
  if constexpr (ROPE) {
    const uint32_t toff = pos * (uint32_t)(2 * D) + lc * 16u;
    cv = ld16(reinterpret_cast<const uint16_t *>(reinterpret_cast<const char *>(p.cos) + toff));
    sv = ld16(reinterpret_cast<const uint16_t *>(reinterpret_cast<const char *>(p.sin) + toff));
  }
  if constexpr (ST == ST_FACTORED) gqv = ld16(p.gq + lc * 8);
  // Every load is issued before the rows' round trip: the stores below are
  // conditional, and without this barrier the compiler sinks the table loads
  // into their branch, behind the wait for the rows.
  asm volatile("" ::: "memory");
  float c[8], sn[8];
  if constexpr (ROPE) {
    // First half: n*c - np*s; second half: n*c + np*s.  Negating s in the
    // first half (a sign flip of the BF16 bits, exact) turns both into
    // n*c + np*s' with the same products and roundings.
    const uint32_t flip = first ? 0x80008000u : 0u;
    sv ^= u32x4_t{flip, flip, flip, flip};
    unpack8(cv, c);
    unpack8(sv, sn);
  }
  float go[8];
  unpack8(g_own, go);
  float gq[8];
  if constexpr (ST == ST_FACTORED) unpack8(gqv, gq);

  // Both rows are computed before either is stored: loads and stores share
  // vmcnt, so a store issued between the rows would make the second row's
  // wait for its load also wait for the first row's store.
  u32x4_t yv[U];
  float invr[U];
#pragma unroll
  for (int i = 0; i < U; ++i) {
    float x[8];
    unpack8(xv[i], x);
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) ss = __fmaf_rn(x[j], x[j], ss);
    ss = row_sum<LPR>(ss);
    const float inv = rsqrt_rn(ss * (1.0f / D) + p.eps);
    invr[i] = inv;
    float y[8];
    if constexpr (ST == ST_FACTORED) {
      // qk:602-609 (K rows): one rounding of x*inv*gk*gq; Q rows keep only inv
#pragma unroll
      for (int j = 0; j < 8; ++j) y[j] = __fmul_rn(__fmul_rn(__fmul_rn(x[j], inv), go[j]), gq[j]);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) y[j] = norm_elem<ST>(x[j], inv, go[j]);
      if constexpr (ROPE) {
#pragma unroll
        for (int j = 0; j < 8; ++j) y[j] = rope_elem<ST>(y[j], partner_f32<LPR>(y[j]), c[j], sn[j], false);
      }
    }
    yv[i] = pack8(y);
    // The rows are finished here, with every lane active: otherwise the
    // compiler sinks their arithmetic into the store branches below, where
    // the partner exchange (DPP, which needs every lane) no longer folds
    // into the multiplies.
    asm volatile("" ::"v"(yv[i]), "v"(invr[i]));
  }
#pragma unroll
  for (int i = 0; i < U; ++i) {
    // a lane past S, or a second head past the tensor's last, stores nothing
    if (!(pvalid && h0 + i < nh)) continue;
    if (ST == ST_FACTORED && is_q) {  // qk:597-601: FP32 inverse RMS per Q row
      if (lc == 0) p.inv[row[i]] = invr[i];
    } else {
      st_row(reinterpret_cast<uint16_t *>(dst + off[i]), yv[i]);
    }
  }
}

template <int D, int ST, bool ROPE, bool ONLY_K, bool VT, int U = ROWS_HPW>
hipError_t launch_rows_t(const RowsParams &p, int64_t blocks, hipStream_t stream) {
  hipLaunchKernelGGL((rows_kernel<D, ST, ROPE, ONLY_K, VT, U>), dim3((unsigned)blocks), dim3(256), 0, stream, p);
  static const std::string name = [] {
    char b[96];
    snprintf(b, sizeof(b), "rows_kernel<%d, %d, %s, %s, %s, %d>", D, ST, tf(ROPE), tf(ONLY_K), tf(VT), U);
    return std::string(b);
  }();
  launch_log_add(reinterpret_cast<const void *>(&rows_kernel<D, ST, ROPE, ONLY_K, VT, U>), name.c_str(), blocks, 256);
  return hipGetLastError();
}

template <int D, int ST, bool ROPE>
hipError_t dispatch_k(const RowsParams &p, bool only_k, hipStream_t s) {
  if constexpr (D == 128 && ST != ST_FACTORED) {
    if (p.vt) {
      const int64_t all = p.row_blocks + p.vt_tiles;
      return only_k ? launch_rows_t<D, ST, ROPE, true, true>(p, all, s) : launch_rows_t<D, ST, ROPE, false, true>(p, all, s);
    }
    if (p.hpw == ROWS_HPW_BIG) return launch_rows_t<D, ST, ROPE, false, false, ROWS_HPW_BIG>(p, p.row_blocks, s);
  }
  return only_k ? launch_rows_t<D, ST, ROPE, true, false>(p, p.row_blocks, s)
                : launch_rows_t<D, ST, ROPE, false, false>(p, p.row_blocks, s);
}

template <int D>
hipError_t dispatch_rows(const RowsParams &p, int style, bool rope, bool only_k, hipStream_t s) {
  switch (style) {
    case ST_HF: return rope ? dispatch_k<D, ST_HF, true>(p, only_k, s) : dispatch_k<D, ST_HF, false>(p, only_k, s);
    case ST_LEGACY:
      return rope ? dispatch_k<D, ST_LEGACY, true>(p, only_k, s) : dispatch_k<D, ST_LEGACY, false>(p, only_k, s);
    case ST_FP32: return rope ? dispatch_k<D, ST_FP32, true>(p, only_k, s) : dispatch_k<D, ST_FP32, false>(p, only_k, s);
    case ST_FACTORED: return dispatch_k<D, ST_FACTORED, false>(p, only_k, s);
  }
  return hipErrorInvalidValue;
}

template <int D>
__global__ __launch_bounds__(256) void transpose_v_kernel(const uint16_t *__restrict__ v, uint16_t *__restrict__ vt,
                                                          int64_t S) {
  transpose_tile<D>(v, vt, S, blockIdx.y, (int64_t)blockIdx.x * 64);
}

}  // namespace

hipError_t launch_transpose_v(const uint16_t *v, uint16_t *vt, int64_t BH, int64_t S, int64_t D, hipStream_t stream) {
  const dim3 grid((unsigned)((S + 63) / 64), (unsigned)BH);
  if (D == 128) {
    hipLaunchKernelGGL((transpose_v_kernel<128>), grid, dim3(256), 0, stream, v, vt, S);
    launch_log_add(reinterpret_cast<const void *>(&transpose_v_kernel<128>), "transpose_v_kernel<128>",
                   (int64_t)grid.x * grid.y, 256);
  } else {
    hipLaunchKernelGGL((transpose_v_kernel<256>), grid, dim3(256), 0, stream, v, vt, S);
    launch_log_add(reinterpret_cast<const void *>(&transpose_v_kernel<256>), "transpose_v_kernel<256>",
                   (int64_t)grid.x * grid.y, 256);
  }
  return hipGetLastError();
}

hipError_t launch_rows(const RowsArgs &a, hipStream_t stream) {
  RowsParams p;
  p.q = a.q; p.k = a.k; p.gq = a.gq; p.gk = a.gk; p.cos = a.cos; p.sin = a.sin;
  p.qn = a.qn; p.kn = a.kn; p.inv = a.inv;
  p.v = a.v; p.vt = a.vt;
  p.S = a.S;
  p.s32 = (uint32_t)a.S;
  p.eps = a.eps;
  // Each tensor has fewer than 2^31 elements (checked at the boundary), so
  // row counts and rows*D fit 32 bits.
  p.heads_q = a.only_k ? 0u : (uint32_t)(a.B * a.Hq);
  p.heads_k = (uint32_t)(a.B * a.Hkv);
  const int64_t rpb = 256 / (a.D / 8);
  p.nblk = (uint32_t)((a.S + rpb - 1) / rpb);
  const int64_t rows = (int64_t)(p.heads_q + p.heads_k) * a.S;
  const bool big_ok = a.D == 128 && !a.only_k && !a.vt && a.style != ST_FACTORED;  // where the 4-head form exists
  const int forced = thread_tuning().rows_heads;
  const bool big_by_shape = (rows >= ROWS_MID_MIN && rows < ROWS_MID_END) ||
                            (a.style == ST_FP32 && rows >= ROWS_BIG && a.S <= ROWS_BIG_MAX_S);
  p.hpw = big_ok && (forced ? forced == ROWS_HPW_BIG : big_by_shape) ? ROWS_HPW_BIG : ROWS_HPW;
  const int64_t units = (p.heads_q + p.hpw - 1) / p.hpw + (p.heads_k + p.hpw - 1) / p.hpw;
  p.row_blocks = (uint32_t)(units * p.nblk);
  p.vt_sblocks = (int)((a.S + 63) / 64);
  p.vt_tiles = a.vt ? a.B * a.Hkv * p.vt_sblocks : 0;
  if (a.vt && a.D != 128) return hipErrorInvalidValue;
  const hipError_t e = a.D == 128 ? dispatch_rows<128>(p, a.style, a.rope, a.only_k, stream)
                                   : dispatch_rows<256>(p, a.style, a.rope, a.only_k, stream);
  launch_log_plan("hpw=%d", (int)p.hpw);
  return e;
}

}  // namespace kfmi
