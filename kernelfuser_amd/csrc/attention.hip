// The general attention kernel (attn_fwd_kernel: any D in {128, 256} and
// GQA ratio, 4 waves = 128 query rows of one head, GEMM1 of tile t+1 issued
// ahead of the softmax and GEMM2 of tile t, lean online softmax with an exact
// redo, split-KV halves at D = 256) and the dispatch of launch_attention over
// the three kernels.  Counterpart of the reference's attention_v2_kernel
// (src/e1_rope_publication_v1.py:608-649) and factored_attention_kernel
// (src/e1_qk_publication_v3.py:612-638).  The arithmetic the kernels share
// (Q prologue, online softmax, MFMA operand layouts, LDS staging, epilogue) is
// in attn_common.h; the ping-pong kernel is in attn_pp.hip, the wide-wave
// kernel in attn_wide.hip.
#include <math.h>

#include <atomic>

#include <cstdio>
#include <string>

#include "attn_common.h"

namespace kfmi {
namespace {

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

  clock_stamp<false>(p.stamps);
  // Two-slot pairing (slot2 > 0): the second slot holds the short causal
  // blocks, whose workgroups have slack; they start about 12k cycles late, so
  // the long blocks of the first slot, which set the kernel's end, stage their
  // tables, Q rows and first tiles without that traffic.  Measured against no
  // delay, alternated on one box: B=1 S=2048 46.5 vs 47.5 us, S=1536 33.6 vs
  // 33.9 us, B=2 S=1024 28.1 vs 28.7 us; 6k cycles gained less at S=2048
  // (46.8 us), 18k cycles lost at B=2 S=1024 (28.8 us).  (s_sleep n waits
  // about 64n cycles.)
  if (CAUSAL && p.slot2 > 0 && (int)blockIdx.x >= p.slot2) {
    __builtin_amdgcn_s_sleep(96);
    __builtin_amdgcn_s_sleep(96);
  }
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
    // Probabilities up to 2^64 keep the row sums finite but can still
    // overflow O when |V| is large.
    bad |= any_not_finite(o);  // no short circuit: a branch here costs the loop registers
    // A lean tile failed somewhere in the workgroup (a logit far above the
    // first tile's row max, or an accumulator that overflowed): every wave
    // redoes the item on the exact path.
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
    clock_stamp<true>(p.stamps);
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
  if (arrived_before == 0) {  // the other half merges
    clock_stamp<true>(p.stamps);
    return;
  }
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
  clock_stamp<true>(p.stamps);
}

template <int D, int BN, bool CAUSAL, int PRO, int ST, bool FK>
const char *fwd_name() {
  static const std::string n = [] {
    char b[96];
    snprintf(b, sizeof(b), "attn_fwd_kernel<%d, %d, %s, %d, %d, %s>", D, BN, tf(CAUSAL), PRO, ST, tf(FK));
    return std::string(b);
  }();
  return n.c_str();
}
template <int D, int BN, bool CAUSAL, int PRO, int ST>
hipError_t launch_t(const AttnParams &p, int kind, int blocks, hipStream_t s) {
  if constexpr (PRO == PRO_NORM || PRO == PRO_NORM_ROPE) {
    if (p.gk) {  // mode 'full': general kernel with the per-tile K prologue
      hipLaunchKernelGGL((attn_fwd_kernel<D, BN, CAUSAL, PRO, ST, true>), dim3(blocks), dim3(256), 0, s, p);
      launch_log_add(reinterpret_cast<const void *>(&attn_fwd_kernel<D, BN, CAUSAL, PRO, ST, true>),
                     fwd_name<D, BN, CAUSAL, PRO, ST, true>(), blocks, 256);
      return hipGetLastError();
    }
  }
  if constexpr (D == 128) {
    if (kind == KFMI_KERNEL_WIDE) return launch_wide(p, CAUSAL, PRO, ST, blocks, s);
    if (kind == KFMI_KERNEL_PINGPONG) return launch_pp(p, CAUSAL, PRO, ST, blocks, s);
  }
  hipLaunchKernelGGL((attn_fwd_kernel<D, BN, CAUSAL, PRO, ST>), dim3(blocks), dim3(256), 0, s, p);
  launch_log_add(reinterpret_cast<const void *>(&attn_fwd_kernel<D, BN, CAUSAL, PRO, ST, false>),
                 fwd_name<D, BN, CAUSAL, PRO, ST, false>(), blocks, 256);
  return hipGetLastError();
}

template <int D, int BN, bool CAUSAL>
hipError_t dispatch_pro(const AttnParams &p, int pro, int st, int kind, int blocks, hipStream_t s) {
  switch (pro) {
    case PRO_NONE: return launch_t<D, BN, CAUSAL, PRO_NONE, ST_FP32>(p, kind, blocks, s);
    case PRO_FACTORED_READ: return launch_t<D, BN, CAUSAL, PRO_FACTORED_READ, ST_FP32>(p, kind, blocks, s);
    case PRO_FACTORED_CALC: return launch_t<D, BN, CAUSAL, PRO_FACTORED_CALC, ST_FP32>(p, kind, blocks, s);
    case PRO_NORM:
      if (st == ST_HF) return launch_t<D, BN, CAUSAL, PRO_NORM, ST_HF>(p, kind, blocks, s);
      if (st == ST_LEGACY) return launch_t<D, BN, CAUSAL, PRO_NORM, ST_LEGACY>(p, kind, blocks, s);
      return launch_t<D, BN, CAUSAL, PRO_NORM, ST_FP32>(p, kind, blocks, s);
    case PRO_NORM_ROPE:
      if (st == ST_HF) return launch_t<D, BN, CAUSAL, PRO_NORM_ROPE, ST_HF>(p, kind, blocks, s);
      if (st == ST_LEGACY) return launch_t<D, BN, CAUSAL, PRO_NORM_ROPE, ST_LEGACY>(p, kind, blocks, s);
      return launch_t<D, BN, CAUSAL, PRO_NORM_ROPE, ST_FP32>(p, kind, blocks, s);
  }
  return hipErrorInvalidValue;
}

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

struct PpGrid {
  int hpg;
  int64_t n_qblocks, npairs, items, units;
  bool xcd_remap, persistent;
};

// Geometry of the ping-pong kernel's grid: items of hpg Q heads per wave
// group (two heads x 128 rows for hpg 1, four heads x 64 rows for hpg 2),
// and whether the persistent long/short pairing applies (causal, the pairs
// of every (long, short) item fill all CUs equally, XCD-remapped heads).
PpGrid pp_grid(int64_t B, int64_t Hq, int64_t Hkv, int64_t S, bool causal, int hpg, int64_t cus) {
  PpGrid g;
  const int64_t G = Hq / Hkv;
  g.hpg = hpg;
  g.n_qblocks = (S + 128 / hpg - 1) / (128 / hpg);
  g.npairs = B * Hkv * (G / (2 * hpg));
  g.xcd_remap = (B * Hkv) % 8 == 0 && g.npairs % 8 == 0;
  g.items = g.n_qblocks * g.npairs;
  g.units = g.npairs * ((g.n_qblocks + 1) / 2);
  g.persistent = causal && g.xcd_remap && cus % 8 == 0 && g.units % cus == 0;
  return g;
}

int pp_heads_for(int64_t Hq, int64_t Hkv) {
  const int t = thread_tuning().pp_heads;
  return t ? t : (Hq / Hkv) % 4 == 0 ? 2 : 1;
}

}  // namespace

// Kernel choice by shape, from the tuning runner's measurements on MI355X
// (every alternative gated and timed per shape).  The ping-pong kernel needs
// D = 128 and an even GQA ratio and runs one 512-thread workgroup per CU;
// below 16 query blocks of 128 rows its per-item Q prologues and few items
// per CU lose to the general kernel (two 4-wave workgroups per CU): B=1
// S=1024 27 vs 33 us, B=8 S=1024 causal 100 vs 99 us (FP32 style) and 109
// vs 105 us (HF style), B=16 S=1024 within 2% either way by style.  The exception is a causal grid
// whose persistent pairs give every CU exactly one (long, short) unit: B=4
// S=1000 runs 51.4-53.1 vs 53.8-54.8 us in the FP32 style (paired ratio
// 1.03-1.04, CI above 1) and ties at 56.5-56.8 us in the HF style.  Units of
// a few tiles do not pay for their items' prologues: B=32 S=128 (one unit
// of 3 tiles per CU) runs 37.7 vs 35.6 us, so the exception needs 8 query
// blocks of 128 rows.  From 16 blocks on
// it wins when its items fill whole rounds of CUs: non-causal, when the item
// count is a multiple of the CU count (S=2048 74.8 vs 78.4 us; S=3072, 1.5
// rounds, 169 vs 156 us for the general kernel); causal, when the persistent
// pairing applies (Qwen3-32B S=2048 78 vs 83 us; Qwen3-8B S=2048, half the
// CUs paired, 61.5 vs 54.2 us) and always from 24 blocks (S=3072 93.7 vs
// 97.2 us, S=4096 141 vs 153 us).  The wide kernel runs only when the
// tuning overrides ask for it: one wave per SIMD issues the softmax's VALU
// work and the MFMA stream by itself, and it measures 5-12% slower than the
// ping-pong kernel from S=3072 on.
int attention_kernel_by_shape(int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t D, bool causal) {
  const int64_t G = Hq / Hkv;
  const int64_t qb128 = (S + 127) / 128;
  if (D != 128 || G % 2 != 0) return KFMI_KERNEL_GENERAL;
  if (causal && qb128 >= 24) return KFMI_KERNEL_PINGPONG;
  const int64_t cus = device_cus();
  const PpGrid g = pp_grid(B, Hq, Hkv, S, causal, pp_heads_for(Hq, Hkv), cus);
  const bool paired = causal && g.persistent && thread_tuning().persistent != 1;
  if (qb128 < 16) return paired && g.units == cus && qb128 >= 8 ? KFMI_KERNEL_PINGPONG : KFMI_KERNEL_GENERAL;
  const bool fills = causal ? paired : g.items % cus == 0;
  return fills ? KFMI_KERNEL_PINGPONG : KFMI_KERNEL_GENERAL;
}

const char *attention_tuning_error(int64_t Hq, int64_t Hkv, int64_t D, bool full) {
  const kfmi_tuning &t = thread_tuning();
  const int64_t G = Hq / Hkv;
  const int k = full ? KFMI_KERNEL_GENERAL : t.attn_kernel;
  if (k == KFMI_KERNEL_PINGPONG && (D != 128 || G % 2 != 0))
    return "the ping-pong kernel needs D == 128 and an even Hq/Hkv";
  if (k == KFMI_KERNEL_WIDE && (D != 128 || G % 4 != 0))
    return "the wide kernel needs D == 128 and Hq/Hkv divisible by 4";
  // wherever the ping-pong kernel may run (forced, or chosen by shape)
  const bool pp_possible = k == KFMI_KERNEL_PINGPONG || (k == KFMI_KERNEL_AUTO && D == 128 && G % 2 == 0);
  if (t.pp_heads == 2 && G % 4 != 0 && pp_possible)
    return "four heads per ping-pong item need Hq/Hkv divisible by 4";
  return nullptr;
}

int attention_kernel(int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t D, bool causal, bool full) {
  if (full) return KFMI_KERNEL_GENERAL;
  const int k = thread_tuning().attn_kernel;
  return k != KFMI_KERNEL_AUTO ? k : attention_kernel_by_shape(B, Hq, Hkv, S, D, causal);
}

}  // namespace kfmi

namespace kfmi {

namespace {


// Split-KV plan for the general kernel at D = 256, which runs one workgroup
// per CU: with fewer work items than CUs, longest-first ordering cannot
// balance a causal grid (the heaviest query block alone sets the time, and
// no co-resident workgroup fills the gap).  Blocks with more key tiles than
// half the maximum are then split into two halves of their key range (the
// second holds the diagonal), and all items are listed longest first.
// Measured with the tuning runner: unsplit grids of 64-192 workgroups gain
// 4-27% (Gemma-3-4B S=2048 57.2 vs 72.6 us), while a grid that already
// fills every CU (Gemma-3-12B S=2048, 256 workgroups) loses 8% (83.1 vs
// 77.0 us), so the plan needs fewer query blocks than CUs.  At D = 128 two
// workgroups share each CU and one already keeps it nearly busy, so the
// extra prologues of a split cost more than the balance gains.

// Workspace layout: a counter region of the same size for every shape (one
// 4-byte arrival counter per split (block, head) pair, at most
// SPLIT_MAX_PAIRS; a plan has fewer than B*Hq*nqb < CUs pairs), then the
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
  if (D != 256 || !causal || nqb < 2 || B * Hq * nqb >= cus) return false;
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
  SplitPlan pl;
  if (!plan_split(B, Hq, S, D, causal, device_cus(), pl)) return 0;
  const int64_t pairs = (int64_t)pl.n_split * B * Hq;
  return SPLIT_COUNTER_BYTES + split_partial_bytes(pairs, D);
}

int64_t attention_workspace_counter_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t D, bool causal) {
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
  p.stamps = nullptr;
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
  const kfmi_tuning &tun = thread_tuning();
  const int kind = attention_kernel(a.B, a.Hq, a.Hkv, a.S, a.D, a.causal, a.gk != nullptr);
  if (kind == KFMI_KERNEL_PINGPONG && a.vt && a.S % 8 == 0) p.vt = a.vt;  // V^T rows must be 16-byte aligned
  int blocks, n_split = 0;
  if (kind == KFMI_KERNEL_PINGPONG || kind == KFMI_KERNEL_WIDE) {
    // items of hpg Q heads per wave group: the wide kernel's four heads x 64
    // rows, or the ping-pong kernel's two heads x 128 rows (hpg 1) or four x
    // 64 (hpg 2)
    const int64_t cus = device_cus();
    const PpGrid g = pp_grid(a.B, a.Hq, a.Hkv, a.S, a.causal, kind == KFMI_KERNEL_WIDE ? 2 : pp_heads_for(a.Hq, a.Hkv),
                             cus);
    p.pp_hpg = g.hpg;
    p.n_qblocks = (int)g.n_qblocks;
    p.xcd_remap = g.xcd_remap ? 1 : 0;
    blocks = (int)g.items;
    // persistent mode when the (long, short) pairs fill every CU equally
    if (g.persistent && tun.persistent != 1) {
      p.pp_units = (int)g.units;
      blocks = (int)cus;
    }
  } else {
    const int nbh = p.B * p.Hq;
    p.xcd_remap = (nbh % 8 == 0 && (p.B * p.Hkv) % 8 == 0) ? 1 : 0;
    blocks = p.n_qblocks * nbh;
    SplitPlan pl;
    if (a.work && tun.split != 1 && plan_split(a.B, a.Hq, a.S, a.D, a.causal, device_cus(), pl)) {
      const int64_t pairs = (int64_t)pl.n_split * nbh;
      if (a.work_bytes >= SPLIT_COUNTER_BYTES + split_partial_bytes(pairs, a.D)) {
        n_split = pl.n_split;
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
  if (tun.clock_stamps) {
    void *st = nullptr;
    const hipError_t se = clock_stamp_buffer(&st);
    if (se != hipSuccess) return se;
    p.stamps = (unsigned long long *)st;
    clock_stamps_recorded(blocks);
  }
  hipError_t e;
  if (a.D == 128) {
    e = a.causal ? dispatch_pro<128, 64, true>(p, a.prologue, a.style, kind, blocks, stream)
                 : dispatch_pro<128, 64, false>(p, a.prologue, a.style, kind, blocks, stream);
  } else {
    e = a.causal ? dispatch_pro<256, 32, true>(p, a.prologue, a.style, KFMI_KERNEL_GENERAL, blocks, stream)
                 : dispatch_pro<256, 32, false>(p, a.prologue, a.style, KFMI_KERNEL_GENERAL, blocks, stream);
  }
  if (kind == KFMI_KERNEL_PINGPONG || kind == KFMI_KERNEL_WIDE)
    launch_log_plan("hpg=%d persistent=%d xcd=%d", p.pp_hpg, p.pp_units > 0 ? 1 : 0, p.xcd_remap);
  else
    launch_log_plan("split=%d pair=%d xcd=%d", n_split, p.slot2 > 0 ? 1 : 0, p.xcd_remap);
  return e;
}

}  // namespace kfmi
