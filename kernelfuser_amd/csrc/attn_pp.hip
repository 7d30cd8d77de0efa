// Ping-pong attention kernel (attn_pp_kernel) and its launcher; shared
// device code in attn_common.h.
#include <cstdio>
#include <string>

#include "attn_common.h"

namespace kfmi {
namespace {

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

  clock_stamp<false>(p.stamps);
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
  clock_stamp<true>(p.stamps);
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

template <bool CAUSAL, int PRO, int ST>
hipError_t launch_pp_t(const AttnParams &p, int blocks, hipStream_t s) {
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

template <bool CAUSAL>
hipError_t launch_pp_c(const AttnParams &p, int pro, int st, int blocks, hipStream_t s) {
  switch (pro) {
    case PRO_NONE: return launch_pp_t<CAUSAL, PRO_NONE, ST_FP32>(p, blocks, s);
    case PRO_FACTORED_READ: return launch_pp_t<CAUSAL, PRO_FACTORED_READ, ST_FP32>(p, blocks, s);
    case PRO_FACTORED_CALC: return launch_pp_t<CAUSAL, PRO_FACTORED_CALC, ST_FP32>(p, blocks, s);
    case PRO_NORM:
      if (st == ST_HF) return launch_pp_t<CAUSAL, PRO_NORM, ST_HF>(p, blocks, s);
      if (st == ST_LEGACY) return launch_pp_t<CAUSAL, PRO_NORM, ST_LEGACY>(p, blocks, s);
      return launch_pp_t<CAUSAL, PRO_NORM, ST_FP32>(p, blocks, s);
    case PRO_NORM_ROPE:
      if (st == ST_HF) return launch_pp_t<CAUSAL, PRO_NORM_ROPE, ST_HF>(p, blocks, s);
      if (st == ST_LEGACY) return launch_pp_t<CAUSAL, PRO_NORM_ROPE, ST_LEGACY>(p, blocks, s);
      return launch_pp_t<CAUSAL, PRO_NORM_ROPE, ST_FP32>(p, blocks, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_pp(const AttnParams &p, bool causal, int pro, int st, int blocks, hipStream_t s) {
  return causal ? launch_pp_c<true>(p, pro, st, blocks, s) : launch_pp_c<false>(p, pro, st, blocks, s);
}

}  // namespace kfmi
