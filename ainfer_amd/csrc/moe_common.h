// moe_common.h - device helpers shared by the gfx950 MoE kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/ainfer_moe.h"

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;

#define WAVE 64

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float((uint32_t)b << 16);
}
// round to nearest even, NaN kept quiet
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
__device__ __forceinline__ float fp16_to_f32(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}
template <int SD>
__device__ __forceinline__ float scale_to_f32(uint16_t s) {
  if constexpr (SD == AINFER_SCALE_FP16)
    return fp16_to_f32(s);
  else
    return bf16_to_f32(s);
}

__device__ __forceinline__ f32x4 mfma_bf16_16x16x32(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c,
                                                 0, 0, 0);
}

// Four packed int4 -> bf16 pairs for one MFMA k-slice.
// d is a dword of 8 nibbles (k offsets 0..7, low nibble first) already
// xor'ed with 0x88888888 so each nibble holds q + 8.  Slice j (0..3) takes
// nibbles j and j+4 into the low/high bf16 halves as 128 + (q + 8): the
// bf16 pattern 0x43NN with N the nibble is exactly 128 + N.
__device__ __forceinline__ uint32_t nib_pair_bf16(uint32_t d, int j) {
  return ((d >> (4 * j)) & 0x000F000Fu) | 0x43004300u;
}

// Index inside a 32-element block of the MFMA-order ("slice-major")
// layout: position p = 8*j + e holds natural k = 4*e + j.
__host__ __device__ __forceinline__ int perm32_pos(int k) {
  return (k & ~31) | (((k & 3) << 3) | ((k & 31) >> 2));
}

// ---- wave64 reductions on the DPP path (no LDS round trip) ---------------
// Inclusive reduction up to lane 63 (quad_perm xor1/xor2, row half-mirror,
// row mirror, row_bcast15, row_bcast31), then a readlane broadcast.
template <typename Op>
__device__ __forceinline__ uint32_t wave_reduce_u32(uint32_t v, Op op) {
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0xB1, 0xF, 0xF, false));
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x4E, 0xF, 0xF, false));
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x141, 0xF, 0xF, false));
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x140, 0xF, 0xF, false));
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x142, 0xA, 0xF, false));
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x143, 0xC, 0xF, false));
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  return wave_reduce_u32(v, [](uint32_t a, uint32_t b) { return a > b ? a : b; });
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
  return wave_reduce_u32(v, [](uint32_t a, uint32_t b) { return a < b ? a : b; });
}
// fp32 -> uint32 whose unsigned order is the float order (-0 < +0 aside)
__device__ __forceinline__ uint32_t ordered_key(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) == 0u) u = 0u;  // -0 ties with +0, as in float compares
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// ---- buffer loads: lanes whose offset is past num_records read 0 ---------
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes,
                                           0x00020000);
}
__device__ __forceinline__ u32x4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
constexpr uint32_t BUF_OOB = 0x80000000u;

// ---- XCD-aware block order -------------------------------------------------
// Workgroups are dispatched round-robin over the 8 XCDs (block b -> XCD b%8),
// each with its own L2.  This bijection hands each XCD a contiguous range of
// logical block ids, so neighbouring work items (which share operands) run
// on the same L2.
constexpr int N_XCD = 8;
__device__ __forceinline__ int xcd_remap(int b, int G) {
  const int q = G / N_XCD, r = G % N_XCD;
  const int xcd = b % N_XCD, idx = b / N_XCD;
  return xcd < r ? xcd * (q + 1) + idx : r * (q + 1) + (xcd - r) * q + idx;
}
