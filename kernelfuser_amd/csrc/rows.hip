// Row preparation kernels for gfx950: per-(token, head) RMSNorm * gamma with
// optional rotate-half RoPE (the reference's prepare_kernel/_rows,
// src/e1_rope_publication_v1.py:550-605) and the factored no-RoPE
// preparation (src/e1_qk_publication_v3.py:592-609).
//
// Memory-bound design:
//  * a D-wide BF16 row is D/8 lanes x 16 bytes (one 16-lane DPP row for D=128),
//    so a wave64 covers 64/(D/8) consecutive positions of one head and its
//    loads/stores are single contiguous runs of 1 KiB;
//  * the sum of squares is reduced with DPP inside the row, the rotate-half
//    partner (column d +/- D/2) is the lane D/16 away (row_ror:8 for D=128);
//  * a wave keeps the cos/sin rows of its positions and both gamma vectors in
//    registers and walks a chunk of heads, so tables are read once per
//    position per head chunk, not once per row;
//  * FP32 internal arithmetic; the rounding points follow the selected style.
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
  int B, Hq_rows, Hq, Hkv;  // Hq_rows = Q heads processed (0 = K rows only); Hq = Q tensor heads
  int heads_per_chunk, n_groups;
  int rows_by;              // grid rows (blockIdx.y) of the row work; VT tiles follow
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
    float p0 = __fmul_rn(n, c), p1 = __fmul_rn(np, s);
    return first ? __fsub_rn(p0, p1) : __fadd_rn(p0, p1);
  }
  float p0 = round_bf16(n * c), p1 = round_bf16(np * s);  // rope:578-579
  return first ? p0 - p1 : p0 + p1;  // rounded to BF16 at the store (rope:580-581)
}

// Raw 16-byte chunk held by the rotate-half partner lane (lane ^ LPR/2).
template <int LPR>
__device__ __forceinline__ u32x4_t partner_chunk(const u32x4_t &x) {
  u32x4_t r;
  if constexpr (LPR == 16) {
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = dpp_u32<DPP_ROW_ROR8>(x[i]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = (uint32_t)__shfl_xor((int)x[i], LPR / 2);
  }
  return r;
}

template <int LPR>
__device__ __forceinline__ float row_sum(float x) {
  x = sum16(x);
  if constexpr (LPR == 32) x += __shfl_xor(x, 16);
  return x;
}

// Heads in flight per lane and the wave count the head chunks aim for,
// tuned on the six-shape sweep (3 and 12288: +2-3% on the B >= 4 shapes
// over 2 and 16384, the same at B=1).
#ifndef KFMI_ROWS_U
#define KFMI_ROWS_U 3
#endif
#ifndef KFMI_ROWS_WAVES
#define KFMI_ROWS_WAVES 12288
#endif
// K rows only (the attention path's preparation launch): fewer waves, each
// covering more heads, so that every wave's table and gamma loads serve at
// least two rows (4.87 against 5.14 us at B=1, S=4096).
#ifndef KFMI_ROWS_WAVES_K
#define KFMI_ROWS_WAVES_K 6144
#endif
#ifndef KFMI_ROWS_NT
#define KFMI_ROWS_NT 1
#endif
__device__ __forceinline__ u32x4_t ld_row(const uint16_t *p) { return KFMI_ROWS_NT ? ld16_nt(p) : ld16(p); }
__device__ __forceinline__ void st_row(uint16_t *p, const u32x4_t &v) {
  if (KFMI_ROWS_NT) st16_nt(p, v); else st16(p, v);
}

template <int D, int ST, bool ROPE, bool ONLY_K, bool VT>
__global__ __launch_bounds__(256) void rows_kernel(RowsParams p) {
  constexpr int LPR = D / 8;     // lanes per row
  constexpr int RPW = 64 / LPR;  // positions per wave
  constexpr int HALF = LPR / 2;
  constexpr int U = KFMI_ROWS_U;  // heads in flight per lane
  if constexpr (VT) {
    // Grid rows past the row work transpose V tiles (same launch).
    if ((int)blockIdx.y >= p.rows_by) {
      const int64_t t = (int64_t)(blockIdx.y - p.rows_by) * gridDim.x + blockIdx.x;
      if (t < p.vt_tiles) transpose_tile<D>(p.v, p.vt, p.S, t / p.vt_sblocks, (t % p.vt_sblocks) * 64);
      return;  // workgroup-uniform
    }
  }
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (wave >= p.B * p.n_groups) return;  // wave-uniform
  const int b = wave / p.n_groups;
  const int64_t pos = (int64_t)(wave % p.n_groups) * RPW + lane / LPR;
  const int lc = lane % LPR;
  const int d0 = lc * 8;
  const int dp = (lc ^ HALF) * 8;  // column of the partner chunk
  const bool valid = pos < p.S;
  const bool first = lc < HALF;
  const int Hq_rows = ONLY_K ? 0 : p.Hq_rows;
  const int H = Hq_rows + p.Hkv;
  const int h_begin = blockIdx.y * p.heads_per_chunk;
  const int h_end = min(H, h_begin + p.heads_per_chunk);
  const u32x4_t zero = {0u, 0u, 0u, 0u};

  float cs[8], sn[8];
  if (ROPE) {
    unpack8(valid ? ld16(p.cos + pos * D + d0) : zero, cs);
    unpack8(valid ? ld16(p.sin + pos * D + d0) : zero, sn);
  }
  const u32x4_t gq_own = Hq_rows ? ld16(p.gq + d0) : zero;
  const u32x4_t gq_par = (Hq_rows && ROPE) ? ld16(p.gq + dp) : zero;
  const u32x4_t gk_own = ld16(p.gk + d0);
  const u32x4_t gk_par = ROPE ? ld16(p.gk + dp) : zero;
  const u32x4_t gq_fac = (ST == ST_FACTORED) ? ld16(p.gq + d0) : zero;

  for (int h0 = h_begin; h0 < h_end; h0 += U) {
    u32x4_t xv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int hh = h0 + u;
      const uint16_t *src = hh < Hq_rows
                                ? p.q + (((int64_t)b * p.Hq + hh) * p.S + pos) * D + d0
                                : p.k + (((int64_t)b * p.Hkv + (hh - Hq_rows)) * p.S + pos) * D + d0;
      xv[u] = (hh < h_end && valid) ? ld_row(src) : zero;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int hh = h0 + u;
      if (hh >= h_end) break;  // wave-uniform
      const bool is_q = hh < Hq_rows;
      float x[8];
      unpack8(xv[u], x);
      float ss = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) ss = __fmaf_rn(x[j], x[j], ss);
      ss = row_sum<LPR>(ss);
      const float inv = rsqrt_rn(ss * (1.0f / D) + p.eps);
      const int64_t row = is_q ? ((int64_t)b * p.Hq + hh) * p.S + pos
                               : ((int64_t)b * p.Hkv + (hh - Hq_rows)) * p.S + pos;
      if constexpr (ST == ST_FACTORED) {
        if (is_q) {  // qk:597-601: FP32 inverse RMS per Q row
          if (valid && lc == 0) p.inv[row] = inv;
        } else {     // qk:602-609: one rounding of x*inv*gk*gq
          float gk[8], gq[8], y[8];
          unpack8(gk_own, gk);
          unpack8(gq_fac, gq);
#pragma unroll
          for (int j = 0; j < 8; ++j) y[j] = __fmul_rn(__fmul_rn(__fmul_rn(x[j], inv), gk[j]), gq[j]);
          if (valid) st_row(p.kn + row * D + d0, pack8(y));
        }
      } else {
        float go[8], y[8];
        unpack8(is_q ? gq_own : gk_own, go);
        if constexpr (ROPE) {
          float xp[8], gp[8];
          unpack8(partner_chunk<LPR>(xv[u]), xp);
          unpack8(is_q ? gq_par : gk_par, gp);
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const float n = norm_elem<ST>(x[j], inv, go[j]);
            const float np = norm_elem<ST>(xp[j], inv, gp[j]);
            y[j] = rope_elem<ST>(n, np, cs[j], sn[j], first);
          }
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j) y[j] = norm_elem<ST>(x[j], inv, go[j]);
        }
        uint16_t *dst = (is_q ? p.qn : p.kn) + row * D + d0;
        if (valid) st_row(dst, pack8(y));
      }
    }
  }
}

template <int D, int ST, bool ROPE, bool ONLY_K, bool VT>
hipError_t launch_rows_t(const RowsParams &p, int blocks_x, int blocks_y, hipStream_t stream) {
  hipLaunchKernelGGL((rows_kernel<D, ST, ROPE, ONLY_K, VT>), dim3(blocks_x, blocks_y), dim3(256), 0, stream, p);
  return hipGetLastError();
}

template <int D, int ST, bool ROPE>
hipError_t dispatch_k(const RowsParams &p, int bx, int by, hipStream_t s) {
  if constexpr (D == 128 && ST != ST_FACTORED) {
    if (p.vt) {
      const int by_all = by + (int)((p.vt_tiles + bx - 1) / bx);
      return p.Hq_rows ? launch_rows_t<D, ST, ROPE, false, true>(p, bx, by_all, s)
                       : launch_rows_t<D, ST, ROPE, true, true>(p, bx, by_all, s);
    }
  }
  return p.Hq_rows ? launch_rows_t<D, ST, ROPE, false, false>(p, bx, by, s)
                   : launch_rows_t<D, ST, ROPE, true, false>(p, bx, by, s);
}

template <int D>
hipError_t dispatch_rows(const RowsParams &p, int style, bool rope, int bx, int by, hipStream_t s) {
  switch (style) {
    case ST_HF: return rope ? dispatch_k<D, ST_HF, true>(p, bx, by, s) : dispatch_k<D, ST_HF, false>(p, bx, by, s);
    case ST_LEGACY: return rope ? dispatch_k<D, ST_LEGACY, true>(p, bx, by, s) : dispatch_k<D, ST_LEGACY, false>(p, bx, by, s);
    case ST_FP32: return rope ? dispatch_k<D, ST_FP32, true>(p, bx, by, s) : dispatch_k<D, ST_FP32, false>(p, bx, by, s);
    case ST_FACTORED: return dispatch_k<D, ST_FACTORED, false>(p, bx, by, s);
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
  } else {
    hipLaunchKernelGGL((transpose_v_kernel<256>), grid, dim3(256), 0, stream, v, vt, S);
  }
  return hipGetLastError();
}

hipError_t launch_rows(const RowsArgs &a, hipStream_t stream) {
  RowsParams p;
  p.q = a.q; p.k = a.k; p.gq = a.gq; p.gk = a.gk; p.cos = a.cos; p.sin = a.sin;
  p.qn = a.qn; p.kn = a.kn; p.inv = a.inv;
  p.v = a.v; p.vt = a.vt;
  p.S = a.S;
  p.B = (int)a.B;
  p.Hq = (int)a.Hq;
  p.Hq_rows = a.only_k ? 0 : (int)a.Hq;
  p.Hkv = (int)a.Hkv;
  p.eps = a.eps;
  const int lpr = (int)a.D / 8;
  const int rpw = 64 / lpr;
  p.n_groups = (int)((a.S + rpw - 1) / rpw);
  const int H = p.Hq_rows + p.Hkv;
  // Split the heads into chunks so the grid holds about the target number of
  // waves when the position count alone does not.
  const int64_t waves = (int64_t)p.B * p.n_groups;
  const int64_t target = a.only_k ? KFMI_ROWS_WAVES_K : KFMI_ROWS_WAVES;
  int chunks = (int)((target + waves - 1) / waves);
  chunks = chunks < 1 ? 1 : (chunks > H ? H : chunks);
  p.heads_per_chunk = (H + chunks - 1) / chunks;
  const int by = (H + p.heads_per_chunk - 1) / p.heads_per_chunk;
  const int bx = (int)((waves + 3) / 4);
  p.rows_by = by;
  p.vt_sblocks = (int)((a.S + 63) / 64);
  p.vt_tiles = a.vt ? a.B * a.Hkv * p.vt_sblocks : 0;
  if (a.vt && a.D != 128) return hipErrorInvalidValue;
  if (a.D == 128) return dispatch_rows<128>(p, a.style, a.rope, bx, by, stream);
  return dispatch_rows<256>(p, a.style, a.rope, bx, by, stream);
}

}  // namespace kfmi
