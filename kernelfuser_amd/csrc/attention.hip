// Causal / non-causal GQA flash-attention prefill on gfx950 bf16 MFMA with a
// fused Q prologue.  Counterpart of the reference's attention_v2_kernel
// (src/e1_rope_publication_v1.py:608-649) and factored_attention_kernel
// (src/e1_qk_publication_v3.py:612-638).
//
// Work decomposition: one workgroup = 4 waves = BM=128 query rows of one
// (batch, Q head); each wave owns 32 query rows for the whole KV sweep.
//
// Transposed formulation (everything stays in registers between the GEMMs):
//   GEMM1  S^T = K . Q^T   A = K tile rows from LDS (ds_read_b128),
//                           B = the wave's Q rows, held in VGPRs as MFMA
//                               B-operands for the whole sweep;
//          the 32x32 accumulator gives every lane ONE query (lane % 32) and 16
//          keys, so the row max / row sum are lane-local plus one
//          v_permlane32_swap with the other half-wave, and the per-query
//          rescale of O is a per-lane scalar;
//   GEMM2  O^T = V^T . P^T A = V^T read from the row-major V tile in LDS with
//                               ds_read_b64_tr_b16 (transpose on read),
//                           B = P^T straight from the GEMM1 accumulator
//                               (exp2, cvt to bf16, no data movement).
// MFMA: v_mfma_f32_32x32x16_bf16.  Operand layouts: A[m][k] -> lane
// m + 32*(k/8), element k%8; B[k][n] -> lane n + 32*(k/8), element k%8;
// C[m][n] -> lane n + 32*((m/4)%2), register (m/8)*4 + m%4.
//
// K/V staging: tiles of BN rows (16 KiB each) are copied HBM -> LDS by the
// buffer unit (buffer_load_dwordx4 ... lds: lane L of a load writes LDS bytes
// base + 16*L), so no VGPRs, no ds_write and no bounds branches are spent on
// staging: rows past S lie outside the buffer descriptor's range and arrive as
// zeros.  Both K and V are double-buffered; the 16-byte chunks of each row are
// XOR-swizzled (K: chunk ^ (row & 7); V: chunk ^ 2*(row & 3)) so the GEMM1
// row reads and the GEMM2 transpose reads are bank-conflict free.
//
// Pipeline (one barrier per KV tile): iteration t issues the copies of K(t+2)
// and V(t+1), then GEMM1 of tile t+1 and the softmax + GEMM2 of tile t, so the
// exp2/max/sum VALU work of tile t overlaps the MFMAs of tile t+1 and each
// copy has a full iteration to land.
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
// masks are applied only on diagonal/tail tiles, waves skip tiles that are
// fully masked for their rows, and the grid issues the longest query blocks
// first.
#include <math.h>

#include "kfmi_device.h"
#include "kfmi_launch.h"

namespace kfmi {
namespace {

struct AttnParams {
  const uint16_t *q, *k, *v, *gq, *cos, *sin;
  uint16_t *out;
  float *inv;
  int64_t S;
  int B, Hq, Hkv, n_qblocks, xcd_remap;
  float c_scale;  // scale*log2(e); for the factored prologues D^-1/2*log2(e)
  float eps;
};

template <int ST>
__device__ __forceinline__ float norm_elem(float x, float inv, float g) {
  if (ST == ST_HF) return round_bf16(round_bf16(x * inv) * g);
  if (ST == ST_LEGACY) return round_bf16(__fmul_rn(__fmul_rn(x, inv), g));
  return __fmul_rn(__fmul_rn(x, inv), g);
}
template <int ST>
__device__ __forceinline__ float rope_elem(float n, float np, float c, float s, bool first) {
  if (ST == ST_FP32) {
    float p0 = __fmul_rn(n, c), p1 = __fmul_rn(np, s);
    return first ? __fsub_rn(p0, p1) : __fadd_rn(p0, p1);
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

// 16 bytes per lane from buffer offset voff + soff into LDS at lds + 16*lane.
// Issued as inline assembly so the compiler does not guard every later LDS
// read with a wait for it; the kernel orders copies and reads itself
// (wait_copies + barrier).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"  // m0 is reserved; it is set right here
__device__ __forceinline__ void copy16_to_lds(const i32x4_t &rsrc, uint32_t lds, uint32_t voff, uint32_t soff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :
               : "s"(lds), "v"(voff), "s"(rsrc), "s"(soff)
               : "memory", "m0");
}
#pragma clang diagnostic pop

// Wait until every copy this wave issued has landed in LDS.
__device__ __forceinline__ void wait_copies() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

constexpr float RESCALE_SLACK = 8.0f;  // log2 units: probabilities stay <= 2^8

template <int D, int BN, bool CAUSAL, int PRO, int ST>
__global__ __launch_bounds__(256, (D == 128 ? 2 : 1)) void attn_fwd_kernel(AttnParams p) {
  constexpr int BM = 128;            // query rows per workgroup (4 waves x 32)
  constexpr int RB = 2 * D;          // bytes per K/V row
  constexpr int TILE = BN * RB;      // bytes per K or V tile
  constexpr int NINST = TILE / 1024; // 1 KiB copies per tile
  constexpr int LPW = NINST / 4;     // copies per wave per tile
  constexpr int RPI = 1024 / RB;     // rows per copy
  constexpr int CPR = D / 8;         // 16-byte chunks per row
  constexpr int NC = D / 16;         // GEMM1 k-steps (16 columns of d)
  constexpr int NDB = D / 32;        // GEMM2 output blocks (32 columns of d)
  constexpr int NKB = BN / 32;       // GEMM1 output blocks (32 keys)
  constexpr int NK16 = BN / 16;      // GEMM2 k-steps (16 keys)
  constexpr int K0 = 0, K1 = TILE, V0 = 2 * TILE, V1 = 3 * TILE;
  static_assert(TILE == 16384 && LPW * 4 == NINST, "tiles are 16 KiB, 4 copies per wave");

  __shared__ __attribute__((aligned(1024))) unsigned char smem[4 * TILE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5;   // half-wave: selects k-group of the MFMA operands
  const int lr = lane & 31;  // query row of this lane within the wave
  const int64_t S = p.S;

  // ---- work item: heaviest query blocks first; KV groups pinned to an XCD ----
  const int nbh = p.B * p.Hq;
  const int bid = blockIdx.x;
  const int rank = bid / nbh;
  const int r = bid - rank * nbh;
  const int qb = CAUSAL ? p.n_qblocks - 1 - rank : rank;
  const int G = p.Hq / p.Hkv;
  int b, h;
  if (p.xcd_remap) {
    // Workgroups are dispatched round-robin over the 8 XCDs (bid % 8).  Map
    // KV group kg to XCD kg % 8 so the G query heads that read the same K/V
    // share one L2.
    const int xcd = r & 7, j = r >> 3;
    const int kg = xcd + 8 * (j / G);
    b = kg / p.Hkv;
    h = (kg - b * p.Hkv) * G + j % G;
  } else {
    b = r / p.Hq;
    h = r - b * p.Hq;
  }
  const int kvh = h / G;
  const int64_t qoff = ((int64_t)b * p.Hq + h) * S;
  const int64_t kvoff = ((int64_t)b * p.Hkv + kvh) * S;
  const uint16_t *qbase = p.q + qoff * D;
  uint16_t *obase = p.out + qoff * D;

  // Buffer descriptors of this head's K and V rows: reads at or past row S
  // return zeros.
  const uint32_t head_bytes = (uint32_t)(S * RB);
  const i32x4_t krs = buffer_rsrc(p.k + kvoff * D, head_bytes);
  const i32x4_t vrs = buffer_rsrc(p.v + kvoff * D, head_bytes);
  const uint32_t lds0 = (uint32_t)reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) unsigned char *)smem);

  // Copy addressing: copy i of this wave fills LDS rows (w*LPW+i)*RPI + lane/CPR,
  // slot lane%CPR, with the source chunk that the swizzle places there.
  uint32_t kvo[LPW], vvo[LPW];
#pragma unroll
  for (int i = 0; i < LPW; ++i) {
    const int row = (w * LPW + i) * RPI + lane / CPR;
    const int slot = lane % CPR;
    kvo[i] = (uint32_t)(row * RB + ((slot ^ (row & 7)) << 4));
    vvo[i] = (uint32_t)(row * RB + ((slot ^ ((row & 3) << 1)) << 4));
  }
  auto copy_k = [&](int t, int buf) {
#pragma unroll
    for (int i = 0; i < LPW; ++i) copy16_to_lds(krs, lds0 + buf + (w * LPW + i) * 1024, kvo[i], (uint32_t)(t * TILE));
  };
  auto copy_v = [&](int t, int buf) {
#pragma unroll
    for (int i = 0; i < LPW; ++i) copy16_to_lds(vrs, lds0 + buf + (w * LPW + i) * 1024, vvo[i], (uint32_t)(t * TILE));
  };

  const int q0 = qb * BM + w * 32;
  const int qrow = q0 + lr;
  const bool qvalid = qrow < S;
  const u32x4_t zero = {0u, 0u, 0u, 0u};

  // ---- KV tile counts ----
  const int64_t kv_end = CAUSAL ? ((int64_t)(qb + 1) * BM < S ? (int64_t)(qb + 1) * BM : S) : S;
  const int nT = (int)((kv_end + BN - 1) / BN);
  const int64_t wave_end = CAUSAL ? ((int64_t)q0 + 32 < S ? (int64_t)q0 + 32 : S) : S;
  const int nTw = q0 < S ? (int)((wave_end + BN - 1) / BN) : 0;  // tiles with any unmasked key

  // Start the first copies before the prologue's own global loads.
  copy_k(0, K0);
  copy_v(0, V0);
  if (nT > 1) copy_k(1, K1);

  // ---- prologue: Q rows -> B operands (optionally RMSNorm + RoPE) ----
  bf16x8_t qreg[NC];
  float cl = p.c_scale;  // logit multiplier of this lane's query row
  {
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
          unpack8(ld16(p.gq + 16 * c + 8 * g), g1);
          unpack8(ld16(p.gq + 16 * c2 + 8 * g), g2);
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            n1[j] = norm_elem<ST>(x1[j], inv, g1[j]);
            n2[j] = norm_elem<ST>(x2[j], inv, g2[j]);
          }
          if constexpr (PRO == PRO_NORM_ROPE) {
            float cs1[8], sn1[8], cs2[8], sn2[8];
            const int64_t trow = qvalid ? (int64_t)qrow * D : 0;
            unpack8(ld16(p.cos + trow + 16 * c + 8 * g), cs1);
            unpack8(ld16(p.sin + trow + 16 * c + 8 * g), sn1);
            unpack8(ld16(p.cos + trow + 16 * c2 + 8 * g), cs2);
            unpack8(ld16(p.sin + trow + 16 * c2 + 8 * g), sn2);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
              y1[j] = rope_elem<ST>(n1[j], n2[j], cs1[j], sn1[j], true);
              y2[j] = rope_elem<ST>(n2[j], n1[j], cs2[j], sn2[j], false);
            }
          } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) { y1[j] = n1[j]; y2[j] = n2[j]; }
          }
          qreg[c] = as_bf16x8(pack8(y1));
          qreg[c2] = as_bf16x8(pack8(y2));
        }
      }
    }
  }

  // ---- LDS read addressing (constant per lane) ----
  // GEMM1: lane reads row 32*kb + lr, chunk 2c + g; with the K swizzle the
  // slot is 8*(c/4) + ((2*(c%4) + g) ^ (lr & 7)).
  uint32_t kra[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) kra[j] = (uint32_t)(lr * RB + (((2 * j + g) ^ (lr & 7)) << 4));
  // GEMM2 transpose reads: 16-lane group supplies rows (lane%16)/4 + 4g of a
  // 16-key step and 4-column runs 16*((lane/16)%2) + 4*(lane%4) of a 32-wide
  // d block; with the V swizzle the slot is 8*(db/2) + ((4*(db%2) + 2*hh + kk) ^ 2m).
  uint32_t vra[2];
  {
    const int m = (lane >> 2) & 3, hh = (lane >> 4) & 1, kk = (lane >> 1) & 1;
    const int row0 = ((lane & 15) >> 2) + 4 * g;
#pragma unroll
    for (int e = 0; e < 2; ++e) vra[e] = (uint32_t)(row0 * RB + (((4 * e + 2 * hh + kk) ^ (2 * m)) << 4) + (lane & 1) * 8);
  }

  f32x16_t o[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) o[db] = f32x16_t{};
  float m_run = -INFINITY;  // reference max of logits (log2 domain)
  float l_run = 0.f;        // this lane's partial row sum

  auto gemm1 = [&](f32x16_t (&s)[NKB], int kbuf) {
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      s[kb] = f32x16_t{};
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const bf16x8_t a =
            *reinterpret_cast<const bf16x8_t *>(smem + kbuf + kb * 32 * RB + kra[c & 3] + (c >> 2) * 128);
        s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qreg[c], s[kb], 0, 0, 0);
      }
    }
  };

  auto softmax_pv = [&](f32x16_t (&s)[NKB], int t, int vbuf) {
    // masks: register i of block kb holds key 32*kb + 8*(i/4) + 4*g + i%4
    const int64_t kt = (int64_t)t * BN;
    const bool need_mask = (CAUSAL && kt + BN - 1 > q0) || (kt + BN > S);
    if (need_mask) {
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int64_t key = kt + 32 * kb + 8 * (i >> 2) + 4 * g + (i & 3);
          if ((CAUSAL && key > qrow) || key >= S) s[kb][i] = -INFINITY;
        }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[kb][i]);
    mx = max_halves(mx) * cl;
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
    float lsum = 0.f;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kb][i], cl, neg_m));
        s[kb][i] = pv;
        lsum += pv;
      }
    l_run += lsum;
    // P^T operands: 16-key step c2 <- registers 8*(c2%2) .. +7 of block c2/2
    bf16x8_t pb[NK16];
#pragma unroll
    for (int c2 = 0; c2 < NK16; ++c2) {
      u32x4_t wv;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        wv[j] = pack_bf16x2(s[c2 >> 1][8 * (c2 & 1) + 2 * j], s[c2 >> 1][8 * (c2 & 1) + 2 * j + 1]);
      pb[c2] = as_bf16x8(wv);
    }
    // GEMM2: O^T[d][query] += V^T . P^T; the A operand's slot j of half g is
    // key 16*c2 + 8*(j/4) + 4*g + j%4, matching the P^T registers above.
#pragma unroll
    for (int c2 = 0; c2 < NK16; ++c2) {
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        const unsigned char *base = smem + vbuf + 16 * c2 * RB + vra[db & 1] + (db >> 1) * 128;
        const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t *)(base));
        const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t *)(base + 8 * RB));
        const bf16x8_t a = __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
        o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pb[c2], o[db], 0, 0, 0);
      }
    }
  };

  // One pipelined iteration; PAR = t % 2 selects the buffers at compile time.
  auto iteration = [&](auto par, int t, f32x16_t (&cur)[NKB], f32x16_t (&nxt)[NKB]) {
    constexpr int PAR = decltype(par)::value;
    constexpr int KNEXT = PAR ? K0 : K1;   // holds K(t+1)
    constexpr int KFREE = PAR ? K1 : K0;   // held K(t), read in the previous iteration
    constexpr int VCUR = PAR ? V1 : V0;    // holds V(t)
    constexpr int VFREE = PAR ? V0 : V1;   // held V(t-1)
    wait_copies();
    __syncthreads();
    if (t + 2 < nT) copy_k(t + 2, KFREE);
    if (t + 1 < nT) copy_v(t + 1, VFREE);
    if (t + 1 < nTw) gemm1(nxt, KNEXT);
    if (t < nTw) softmax_pv(cur, t, VCUR);
  };

  f32x16_t sa[NKB], sb[NKB];
  wait_copies();
  __syncthreads();
  if (nTw > 0) gemm1(sa, K0);
  for (int t = 0;;) {
    iteration(std::integral_constant<int, 0>{}, t, sa, sb);
    if (++t >= nT) break;
    iteration(std::integral_constant<int, 1>{}, t, sb, sa);
    if (++t >= nT) break;
  }

  // ---- epilogue: O = O^T / l, BF16 rows ----
  const float l_tot = sum_halves(l_run);
  if (qvalid) {
    const float rl = __fdiv_rn(1.0f, l_tot);
    uint16_t *orow = obase + (int64_t)qrow * D;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        u32x2_t wv;
        wv[0] = pack_bf16x2(o[db][4 * q4 + 0] * rl, o[db][4 * q4 + 1] * rl);
        wv[1] = pack_bf16x2(o[db][4 * q4 + 2] * rl, o[db][4 * q4 + 3] * rl);
        *reinterpret_cast<u32x2_t *>(orow + 32 * db + 8 * q4 + 4 * g) = wv;
      }
  }
}

template <int D, int BN, bool CAUSAL, int PRO, int ST>
hipError_t launch_t(const AttnParams &p, int blocks, hipStream_t s) {
  hipLaunchKernelGGL((attn_fwd_kernel<D, BN, CAUSAL, PRO, ST>), dim3(blocks), dim3(256), 0, s, p);
  return hipGetLastError();
}

template <int D, int BN, bool CAUSAL>
hipError_t dispatch_pro(const AttnParams &p, int pro, int st, int blocks, hipStream_t s) {
  switch (pro) {
    case PRO_NONE: return launch_t<D, BN, CAUSAL, PRO_NONE, ST_FP32>(p, blocks, s);
    case PRO_FACTORED_READ: return launch_t<D, BN, CAUSAL, PRO_FACTORED_READ, ST_FP32>(p, blocks, s);
    case PRO_FACTORED_CALC: return launch_t<D, BN, CAUSAL, PRO_FACTORED_CALC, ST_FP32>(p, blocks, s);
    case PRO_NORM:
      if (st == ST_HF) return launch_t<D, BN, CAUSAL, PRO_NORM, ST_HF>(p, blocks, s);
      if (st == ST_LEGACY) return launch_t<D, BN, CAUSAL, PRO_NORM, ST_LEGACY>(p, blocks, s);
      return launch_t<D, BN, CAUSAL, PRO_NORM, ST_FP32>(p, blocks, s);
    case PRO_NORM_ROPE:
      if (st == ST_HF) return launch_t<D, BN, CAUSAL, PRO_NORM_ROPE, ST_HF>(p, blocks, s);
      if (st == ST_LEGACY) return launch_t<D, BN, CAUSAL, PRO_NORM_ROPE, ST_LEGACY>(p, blocks, s);
      return launch_t<D, BN, CAUSAL, PRO_NORM_ROPE, ST_FP32>(p, blocks, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_attention(const AttnArgs &a, hipStream_t stream) {
  constexpr double LOG2E = 1.4426950408889634;
  AttnParams p;
  p.q = a.q; p.k = a.k; p.v = a.v; p.gq = a.gq; p.cos = a.cos; p.sin = a.sin;
  p.out = a.out; p.inv = a.inv;
  p.S = a.S;
  p.B = (int)a.B; p.Hq = (int)a.Hq; p.Hkv = (int)a.Hkv;
  p.eps = a.eps;
  const bool factored = a.prologue == PRO_FACTORED_READ || a.prologue == PRO_FACTORED_CALC;
  // rope:636 SCALE*log2e; qk:621 D**-.5*log2e (both formed in double, then FP32)
  p.c_scale = (float)((factored ? 1.0 / sqrt((double)a.D) : a.scale) * LOG2E);
  const int BM = 128;
  p.n_qblocks = (int)((a.S + BM - 1) / BM);
  const int nbh = p.B * p.Hq;
  p.xcd_remap = (nbh % 8 == 0 && (p.B * p.Hkv) % 8 == 0) ? 1 : 0;
  const int blocks = p.n_qblocks * nbh;
  if (a.D == 128) {
    return a.causal ? dispatch_pro<128, 64, true>(p, a.prologue, a.style, blocks, stream)
                    : dispatch_pro<128, 64, false>(p, a.prologue, a.style, blocks, stream);
  }
  return a.causal ? dispatch_pro<256, 32, true>(p, a.prologue, a.style, blocks, stream)
                  : dispatch_pro<256, 32, false>(p, a.prologue, a.style, blocks, stream);
}

}  // namespace kfmi
