// Shared device/host helpers for the gfx950 varlen kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "scree_hip.h"

namespace scree {

// ------------------------------------------------------------------ errors
// Thread-local message for scree_last_error(); set by host-side validation.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int check_launch(const char* what);

// ------------------------------------------------------------------- types
typedef _Float16 f16;
typedef __bf16 bf16;
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

template <typename T> struct VecT;
template <> struct VecT<f16> { typedef f16x8 x8; typedef f16x4 x4; typedef f16x2 x2; };
template <> struct VecT<bf16> { typedef bf16x8 x8; typedef bf16x4 x4; typedef bf16x2 x2; };

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(f16 v) { return (float)v; }
__device__ __forceinline__ float to_f32(bf16 v) { return (float)v; }

template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ f16 from_f32<f16>(float v) { return (f16)v; }
template <> __device__ __forceinline__ bf16 from_f32<bf16>(float v) { return (bf16)v; }

// Two floats -> one 32-bit word of two 16-bit values, round to nearest even
// (v_cvt_pk_f16_f32 / v_cvt_pk_bf16_f32 on gfx950).
template <typename T> __device__ __forceinline__ uint32_t pack2(float a, float b);
template <> __device__ __forceinline__ uint32_t pack2<f16>(float a, float b) {
  f16x2 h = {(f16)a, (f16)b};
  return __builtin_bit_cast(uint32_t, h);
}
template <> __device__ __forceinline__ uint32_t pack2<bf16>(float a, float b) {
  bf16x2 h = {(bf16)a, (bf16)b};
  return __builtin_bit_cast(uint32_t, h);
}

// 16-bit element `i` (0/1) of a 32-bit word as float.
template <typename T> __device__ __forceinline__ float half_at(uint32_t w, int i);
template <> __device__ __forceinline__ float half_at<f16>(uint32_t w, int i) {
  uint16_t u = (uint16_t)(i ? (w >> 16) : (w & 0xffffu));
  return (float)__builtin_bit_cast(f16, u);
}
template <> __device__ __forceinline__ float half_at<bf16>(uint32_t w, int i) {
  return __builtin_bit_cast(float, i ? (w & 0xffff0000u) : (w << 16));
}

// Element e of a 16-byte vector of T, as float.
template <typename T> __device__ __forceinline__ float elem(const uint4& v, int e);
template <> __device__ __forceinline__ float elem<float>(const uint4& v, int e) {
  uint32_t w = e == 0 ? v.x : e == 1 ? v.y : e == 2 ? v.z : v.w;
  return __builtin_bit_cast(float, w);
}
template <> __device__ __forceinline__ float elem<f16>(const uint4& v, int e) {
  uint32_t w = (e >> 1) == 0 ? v.x : (e >> 1) == 1 ? v.y : (e >> 1) == 2 ? v.z : v.w;
  return half_at<f16>(w, e & 1);
}
template <> __device__ __forceinline__ float elem<bf16>(const uint4& v, int e) {
  uint32_t w = (e >> 1) == 0 ? v.x : (e >> 1) == 1 ? v.y : (e >> 1) == 2 ? v.z : v.w;
  return half_at<bf16>(w, e & 1);
}

// Pack 16/sizeof(T) floats into a 16-byte vector of T.
template <typename T> __device__ __forceinline__ uint4 pack16(const float* f);
template <> __device__ __forceinline__ uint4 pack16<float>(const float* f) {
  return make_uint4(__builtin_bit_cast(uint32_t, f[0]), __builtin_bit_cast(uint32_t, f[1]),
                    __builtin_bit_cast(uint32_t, f[2]), __builtin_bit_cast(uint32_t, f[3]));
}
template <> __device__ __forceinline__ uint4 pack16<f16>(const float* f) {
  return make_uint4(pack2<f16>(f[0], f[1]), pack2<f16>(f[2], f[3]), pack2<f16>(f[4], f[5]),
                    pack2<f16>(f[6], f[7]));
}
template <> __device__ __forceinline__ uint4 pack16<bf16>(const float* f) {
  return make_uint4(pack2<bf16>(f[0], f[1]), pack2<bf16>(f[2], f[3]), pack2<bf16>(f[4], f[5]),
                    pack2<bf16>(f[6], f[7]));
}

__device__ __forceinline__ uint4 ld16(const void* p) { return *reinterpret_cast<const uint4*>(p); }
__device__ __forceinline__ void st16(void* p, const uint4& v) { *reinterpret_cast<uint4*>(p) = v; }

// Streaming (non-temporal) 16-byte accesses for data touched once: they bypass
// cache allocation and sustain ~6.5 TB/s on MI355X versus ~5.9 TB/s plain.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld16_nt(const void* p) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void st16_nt(void* p, const uint4& v) {
  const u32x4 u = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(u, reinterpret_cast<u32x4*>(p));
}

// ------------------------------------------------------------- reductions
__device__ __forceinline__ float wave_sum_last(float v);
// Sum of v over the wave, in every lane (the DPP sum read back from lane 63
// as a wave-uniform value).
__device__ __forceinline__ float wave_sum(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wave_sum_last(v)), 63));
}

// Sum of v over the wave, complete in lane 63 only (other lanes hold partial
// sums): DPP row shifts add each row of 16 lanes into its last lane, then
// row broadcasts carry rows 0 and 2 into rows 1 and 3 and row 1 into rows 2
// and 3 -- VALU operations only, where wave_sum's shuffles go through LDS.
__device__ __forceinline__ float wave_sum_last(float v) {
  // dpp_ctrl: row_shr:n = 0x110 + n, row_bcast:15 = 0x142, row_bcast:31 = 0x143
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x111, 0xf, 0xf, true));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x112, 0xf, 0xf, true));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x114, 0xf, 0xf, true));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x118, 0xf, 0xf, true));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x142, 0xa, 0xf, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x143, 0xc, 0xf, false));
  return v;
}

// --------------------------------------------------------------------- MFMA
// C(32x32, f32) += A(32x16) * B(16x32); lane l holds A row l%32 / B column
// l%32 with k = 8*(l/32) .. +7; C element i of lane l is row
// 8*(i/4) + 4*(l/32) + i%4, column l%32.
__device__ __forceinline__ f32x16 mfma32(const f16x8& a, const f16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma32(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

}  // namespace scree
