// Device helpers shared by the gfx950 kernels: BF16 conversion, DPP and
// cross-half lane exchange, 16-byte memory access, MFMA operand types.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kfmi {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

typedef __attribute__((address_space(3))) i16x4_t lds_i16x4_t;

// ---- BF16 <-> FP32 -------------------------------------------------------
__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Round-to-nearest-even FP32 -> BF16 (hardware v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  f32x2_t f = {lo, hi};
  bf16x2_t h = __builtin_convertvector(f, bf16x2_t);
  return __builtin_bit_cast(uint32_t, h);
}
__device__ __forceinline__ float round_bf16(float x) {
  return bf_lo(pack_bf16x2(x, 0.0f) & 0xffffu);
}

__device__ __forceinline__ void unpack8(const u32x4_t &w, float (&f)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = bf_lo(w[i]);
    f[2 * i + 1] = bf_hi(w[i]);
  }
}
__device__ __forceinline__ u32x4_t pack8(const float (&f)[8]) {
  u32x4_t w;
#pragma unroll
  for (int i = 0; i < 4; ++i) w[i] = pack_bf16x2(f[2 * i], f[2 * i + 1]);
  return w;
}

// ---- memory ----------------------------------------------------------------
__device__ __forceinline__ u32x4_t ld16(const uint16_t *p) {
  return *reinterpret_cast<const u32x4_t *>(p);
}
__device__ __forceinline__ void st16(uint16_t *p, const u32x4_t &v) {
  *reinterpret_cast<u32x4_t *>(p) = v;
}
// Streaming (nontemporal) variants for data touched once: on gfx950 these
// keep single-use rows from displacing reused lines in L2 and raise copy-like
// kernels from ~5.5 to ~6.2 TB/s.
__device__ __forceinline__ u32x4_t ld16_nt(const uint16_t *p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p));
}
__device__ __forceinline__ void st16_nt(uint16_t *p, const u32x4_t &v) {
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4_t *>(p));
}

// ---- lane exchange ---------------------------------------------------------
// DPP controls (GCN/CDNA encoding).
enum : int {
  DPP_QUAD_XOR1 = 0xB1,  // quad_perm [1,0,3,2]
  DPP_QUAD_XOR2 = 0x4E,  // quad_perm [2,3,0,1]
  DPP_ROW_ROR8 = 0x128,  // row_ror:8 (lane i <- lane (i+8) mod 16 within a row of 16)
  DPP_ROW_MIRROR = 0x140,
  DPP_ROW_HALF_MIRROR = 0x141,
};

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, 0xf, 0xf, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
  return __uint_as_float(dpp_u32<CTRL>(__float_as_uint(x)));
}

// Sum over each aligned group of 16 lanes (result in every lane of the group).
__device__ __forceinline__ float sum16(float x) {
  x += dpp_f32<DPP_QUAD_XOR1>(x);
  x += dpp_f32<DPP_QUAD_XOR2>(x);
  x += dpp_f32<DPP_ROW_HALF_MIRROR>(x);
  x += dpp_f32<DPP_ROW_MIRROR>(x);
  return x;
}

// Value held by lane (l ^ 32): v_permlane32_swap(x, x) returns
// r0 = [x0..x31, x0..x31] and r1 = [x32..x63, x32..x63].
__device__ __forceinline__ float xor32(float x, int lane) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(lane < 32 ? r[1] : r[0]);
}
__device__ __forceinline__ float sum_halves(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float max_halves(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Correctly rounded 1/sqrt(x): sqrt and divide both round-to-nearest, the
// same two steps as torch's CPU rsqrt.
__device__ __forceinline__ float rsqrt_rn(float x) { return __fdiv_rn(1.0f, __fsqrt_rn(x)); }

}  // namespace kfmi
