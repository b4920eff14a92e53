// mgi_common.h -- device helpers shared by the gfx950 kernels of
// libminivllm_hip.so: element storage types, exact/rounded conversions,
// 16-byte fragment loads and wavefront row reductions built on DPP.
//
// Written for CDNA4 (gfx950, wave64) only.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mgi {

// Storage types. bf16 and f16 are carried as raw 16-bit patterns so copies
// stay bit-exact and conversions are explicit.
struct bf16_t { uint16_t bits; };
struct f16_t { uint16_t bits; };

// ---------------------------------------------------------------- conversions

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}
// Low / high bf16 of a packed pair (element 2i in the low half, 2i+1 high).
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// float -> bf16, round to nearest even; every NaN becomes 0x7FC0 (the same
// result as torch's float -> bfloat16 cast).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float f16_to_f32(uint16_t bits) {
  return (float)__builtin_bit_cast(_Float16, bits);
}
// float -> f16 with the hardware conversion (round to nearest even).
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

template <typename T> struct Elem;
template <> struct Elem<float> {
  static constexpr int bytes = 4;
  __device__ static float load(const float* p) { return *p; }
  __device__ static void store(float* p, float x) { *p = x; }
};
template <> struct Elem<bf16_t> {
  static constexpr int bytes = 2;
  __device__ static float load(const bf16_t* p) { return bf16_to_f32(p->bits); }
  __device__ static void store(bf16_t* p, float x) { p->bits = f32_to_bf16(x); }
};
template <> struct Elem<f16_t> {
  static constexpr int bytes = 2;
  __device__ static float load(const f16_t* p) { return f16_to_f32(p->bits); }
  __device__ static void store(f16_t* p, float x) { p->bits = f32_to_f16(x); }
};

// ------------------------------------------------------------ index loading

// Loads element i of an int32 or int64 index array (wave-uniform when the
// address is uniform, so the compiler emits scalar loads).
__device__ __forceinline__ int64_t load_index(const void* p, int is64, int64_t i) {
  return is64 ? ((const int64_t*)p)[i] : (int64_t)((const int32_t*)p)[i];
}

// -------------------------------------------------------------- DPP / swizzle

// DPP controls (gfx9 encoding).
constexpr int DPP_QUAD_XOR1 = 0xB1;   // quad_perm:[1,0,3,2]
constexpr int DPP_QUAD_XOR2 = 0x4E;   // quad_perm:[2,3,0,1]
constexpr int DPP_ROW_HALF_MIRROR = 0x141;
constexpr int DPP_ROW_MIRROR = 0x140;

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true));
}

// Exchange with lane ^ 16 inside each 32-lane half (ds_swizzle bitmask mode:
// and_mask 0x1F, or_mask 0, xor_mask 0x10).
__device__ __forceinline__ float swizzle_xor16(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, x), 0x401F));
}

struct SumOp {
  __device__ static float apply(float x, float y) { return x + y; }
};
struct MaxOp {
  __device__ static float apply(float x, float y) { return fmaxf(x, y); }
};

// Reduction over aligned groups of G lanes (G in {1,2,4,8,16,32}); every
// lane of the group receives the result. Within a 16-lane DPP row the partner
// patterns mirror, half-mirror, quad xor2, quad xor1 combine all 16 inputs.
template <int G, typename Op = SumOp>
__device__ __forceinline__ float group_reduce(float x) {
  if constexpr (G >= 16) x = Op::apply(x, dpp<DPP_ROW_MIRROR>(x));
  if constexpr (G >= 8) x = Op::apply(x, dpp<DPP_ROW_HALF_MIRROR>(x));
  if constexpr (G >= 4) x = Op::apply(x, dpp<DPP_QUAD_XOR2>(x));
  if constexpr (G >= 2) x = Op::apply(x, dpp<DPP_QUAD_XOR1>(x));
  if constexpr (G >= 32) x = Op::apply(x, swizzle_xor16(x));
  return x;
}

template <int G>
__device__ __forceinline__ float group_sum(float x) { return group_reduce<G, SumOp>(x); }

// Full 64-lane reductions, result in every lane.
__device__ __forceinline__ float wave_sum(float x) {
  x = group_reduce<32, SumOp>(x);
  return x + __shfl_xor(x, 32, 64);
}
__device__ __forceinline__ float wave_max(float x) {
  x = group_reduce<32, MaxOp>(x);
  return fmaxf(x, __shfl_xor(x, 32, 64));
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ------------------------------------------------------------ buffer loads
// Raw buffer descriptor over `base` (gfx9-family dword3: 32-bit data format,
// no swizzle). Offsets used with it stay below 2^31 (checked on the host), so
// num_records is set to the maximum and never clips a load.
constexpr int kBufferDword3 = 0x00020000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, -1, kBufferDword3);
}

// Cache policy of the streaming loads: NT (non-temporal, cache-policy bit 1).
// Decode reads every K/V byte once per call; marking those lines
// non-temporal raised the decode kernel's HBM throughput on MI355X from
// 73.7% to 79.0% of 8 TB/s (B=64, contexts 512-4096, bf16) and from 75.5% to
// 82.3% for 32k-128k contexts.
constexpr int kStreamCachePolicy = 2;

// 16-byte streaming load at base + soffset (uniform) + voffset (per lane).
__device__ __forceinline__ uint4 buffer_load16(__amdgpu_buffer_rsrc_t rs, uint32_t voffset,
                                               uint32_t soffset) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)voffset, (int)soffset,
                                                                          kStreamCachePolicy));
}

}  // namespace mgi
