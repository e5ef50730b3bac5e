// moe_common.h - device helpers shared by the gfx950 MoE kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <type_traits>
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

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// 16 blocks of D (4x4) += A (4x4) B (4x4), bf16 in, fp32 out.  Block b:
// A row i in lane 4b + i, B column j in lane 4b + j (register = k), D
// element (i, j) in lane 4b + j, register i.
__device__ __forceinline__ f32x4 mfma_bf16_4x4x4(s16x4 a, s16x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(a, b, c, 0, 0, 0);
}

// Sums over the lanes that differ only in the bits of lane mask M and below
// (down to bit 2), halving the values a lane holds at each bit: the lane
// with the bit clear keeps the lower half and receives its partner's lower
// half, the other the upper.  Bits 5 and 4 swap through permlane32/16_swap,
// bits 3 and 2 through ds_swizzle.
template <int N, int M>
struct HalveSum {
  // one halving step over lane mask M: v[0, N/2) <- kept half + partner's
  static __device__ __forceinline__ void step(float *v, int lane) {
    constexpr int h = N / 2;
#pragma unroll
    for (int i = 0; i < h; ++i) {
      if constexpr (M == 32 || M == 16) {
        const u32x2 r = M == 32 ? __builtin_amdgcn_permlane32_swap(__float_as_uint(v[i]),
                                                                   __float_as_uint(v[h + i]),
                                                                   false, false)
                                : __builtin_amdgcn_permlane16_swap(__float_as_uint(v[i]),
                                                                   __float_as_uint(v[h + i]),
                                                                   false, false);
        v[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
      } else {
        const bool up = lane & M;
        const float keep = up ? v[h + i] : v[i], send = up ? v[i] : v[h + i];
        v[i] = keep + __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(send),
                                                                 (M << 10) | 0x1F));
      }
    }
  }
  static __device__ __forceinline__ void run(float *v, int lane) {
    step(v, lane);
    HalveSum<N / 2, M / 2>::run(v, lane);
  }
};
template <int N>
struct HalveSum<N, 2> {
  static __device__ __forceinline__ void run(float *, int) {}
};

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
// sum over the 64 lanes of an fp64 value, in every lane, on the DPP path
// (the same steps as wave_reduce_u32; masked-off rows add 0).  The order of
// the additions is fixed but is not the xor butterfly's: only for sums whose
// result does not depend on the order (rms_mean_f's exact cases).
__device__ __forceinline__ double wave_sum_f64(double v) {
  auto step = [&](auto ctrl_c, auto rmask_c) {
    constexpr int CTRL = decltype(ctrl_c)::value, RMASK = decltype(rmask_c)::value;
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, RMASK, 0xF, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, RMASK, 0xF, false);
    v += __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
  };
  step(std::integral_constant<int, 0xB1>(), std::integral_constant<int, 0xF>());
  step(std::integral_constant<int, 0x4E>(), std::integral_constant<int, 0xF>());
  step(std::integral_constant<int, 0x141>(), std::integral_constant<int, 0xF>());
  step(std::integral_constant<int, 0x140>(), std::integral_constant<int, 0xF>());
  step(std::integral_constant<int, 0x142>(), std::integral_constant<int, 0xA>());
  step(std::integral_constant<int, 0x143>(), std::integral_constant<int, 0xC>());
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, 63);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), 63);
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}
// inclusive prefix sum over the 64 lanes (all active): Hillis-Steele inside
// each row of 16 lanes by DPP row shifts, then the row totals carried across
// rows by row_bcast:15 / row_bcast:31
__device__ __forceinline__ int wave_scan_incl(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);  // row_bcast:15 -> rows 1, 3
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);  // row_bcast:31 -> rows 2, 3
  return v;
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

// ---- device-coherent accesses ----------------------------------------------
// The L2 of each XCD is write-back and not coherent with the other XCDs'.
// Data one workgroup hands to another inside a kernel is written with sc1
// stores (written through to the device coherence point) and read with sc1
// loads, and a wait for the stores' completion precedes the counter atomic
// that publishes them.  This replaces agent-scope release/acquire fences,
// which write back or invalidate a whole L2 (about 20 ns each, serialised).
constexpr int CPOL_SC1 = 16;  // cache-policy operand of the buffer builtins
__device__ __forceinline__ uint16_t ld_dev_u16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, CPOL_SC1);
}
__device__ __forceinline__ void st_dev_u16(__amdgpu_buffer_rsrc_t r, uint32_t off, uint16_t v) {
  __builtin_amdgcn_raw_buffer_store_b16(v, r, off, 0, CPOL_SC1);
}
template <typename V>
__device__ __forceinline__ V ld_dev(const V *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename V>
__device__ __forceinline__ void st_dev(V *p, V v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// threadIdx.x, opaque to the optimiser: in a persistent kernel's loops it
// keeps lane-dependent addresses from being hoisted out of the loop and held
// live (spilled) across every phase.  No instructions.
__device__ __forceinline__ int tid_opaque() {
  int t = threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}

// every store this wave issued has completed
__device__ __forceinline__ void wait_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

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

// MFMA-order copy of one token row (position 8*j+e <- k = 4*e+j inside every
// 32-element block) and, when xsum is non-null, its 128-wide group sums.
// RMSNorm applied on the fly (the decode routing kernel at T <= 16, so a
// block needs no separate RMSNorm launch): the per-token scale and the
// normalized bf16 values are bit-identical to k_rmsnorm (moe_route.hip).
struct NormIn {
  const uint16_t *w;  // norm weight [H] bf16, or null (weight 1)
  int mode;           // AINFER_NORM_PLAIN / AINFER_NORM_ONE_PLUS
  float eps;
  int on;             // 0: x is used as given
};

// float(ss / H) of an RMSNorm row whose fp64 sum of squares is tot, when that
// float is the same for every summation order of the squares.  The reference
// sums sequentially for N != 5120 and as a 256-lane tree for N = 5120
// (tools/cmdlist/kernels.cpp:86-107).  Two sufficient tests:
//  1. exact sums.  A bf16 x = M * 2^(e - 134) (M < 256 an integer, e the
//     exponent field, 1 for subnormals), so x^2 is a multiple of
//     q = 2^(2 * emin - 268), emin the smallest exponent field of the row's
//     non-zero elements.  Every partial sum in any order is a multiple of q
//     no larger than the total; when the total is below 2^53 * q all of them
//     are representable, no addition rounds, and every order gives tot
//     exactly.  bf16 rows usually pass this (their squares have 16-bit
//     significands), and they are also the rows whose tot / H tends to fall
//     on a float rounding midpoint, where test 2 must fail.
//  2. rounding that cannot matter.  Any order of H non-negative terms lies
//     within (H-1)*2^-53*(1+tiny) of the exact sum (recursive-summation bound),
//     so two orders differ by less than H*2^-52 relative and the quotients by
//     H by less than (H+8)*2^-52.  If both ends of that interval around tot/H
//     round to one float, every order gives that float.
// Otherwise it returns false and the caller sums sequentially (rows that
// hold both tiny and large elements and land within 2^-40 of a midpoint).
__device__ __forceinline__ bool rms_mean_f(double tot, int emin, int H, float &mean) {
  const double d = tot / H;
  mean = (float)d;
  if (emin > 0 && tot < __builtin_ldexp(1.0, 2 * emin - 268 + 53)) return true;
  const double m = (double)(H + 8) * 0x1p-52;
  return (float)(d * (1.0 - m)) == (float)(d * (1.0 + m));
}

// exponent field of a bf16 for rms_mean_f's quantum: 1 for subnormals, a
// large value for zeros (they add nothing)
__device__ __forceinline__ int bf16_qexp(uint16_t u) {
  const int e = (u >> 7) & 0xFF;
  return (u & 0x7FFF) == 0 ? 0x7FFF : (e == 0 ? 1 : e);
}

// Sequential fp64 sum of squares of a bf16 row (the reference order for
// N != 5120): the rare fallback of rms_mean_f, run by one lane.  Loads are
// issued 16 elements at a time; the additions stay in element order.
__device__ __forceinline__ double row_sumsq_seq(const uint16_t *__restrict__ xr,
                                                          int H) {
  double ss = 0.0;
  int j = 0;
  if (((uintptr_t)xr & 15) == 0)
    for (; j + 16 <= H; j += 16) {
      const u32x4 a = *(const u32x4 *)(xr + j), b = *(const u32x4 *)(xr + j + 8);
      const uint32_t w[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const double v = (double)bf16_to_f32((uint16_t)(w[i] >> (16 * h)));
          ss += v * v;
        }
    }
  for (; j < H; ++j) {
    const double v = (double)bf16_to_f32(xr[j]);
    ss += v * v;
  }
  return ss;
}

// inv = 1 / sqrt(mean + eps) from a wave's fp64 sum of squares of row xr in any
// order (tot, wave-uniform) and the smallest exponent field emin: the mean is
// the reference's whenever rms_mean_f proves it, else the row is re-summed
// sequentially by lane 0.
__device__ __forceinline__ float rms_inv_finish(double tot, int emin,
                                                const uint16_t *__restrict__ xr, int H, float eps,
                                                int lane) {
  float mean;
  if (!rms_mean_f(tot, emin, H, mean)) {  // wave-uniform
    double ss = 0.0;
    if (lane == 0) ss = row_sumsq_seq(xr, H);
    mean = (float)(__shfl(ss, 0, 64) / H);
  }
  return 1.0f / sqrtf(mean + eps);
}

// Partial fp64 sum of squares and packed exponent key of one 16-byte chunk
// of bf16 (8 elements): squares of bf16 values are exact in fp64 (fma ==
// add of the square); the key is max(exponent field, 1) << 7 per element,
// zeros included as exponent 1 (a smaller emin only makes rms_mean_f's
// exactness test stricter, so it stays a sufficient test).
typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void sumsq_chunk(const u32x4 &v, double (&p4)[4], u16x2_t &ek) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint32_t d = v[q];
    const double lo = (double)__uint_as_float(d << 16);
    const double hi = (double)__uint_as_float(d & 0xFFFF0000u);
    p4[q] = __builtin_fma(lo, lo, p4[q]);
    p4[q] = __builtin_fma(hi, hi, p4[q]);
    const u16x2_t e2 = __builtin_bit_cast(u16x2_t, d & 0x7F807F80u);
    ek = __builtin_elementwise_min(ek, __builtin_elementwise_max(e2, u16x2_t{0x80, 0x80}));
  }
}
__device__ __forceinline__ int ek_emin(u16x2_t ek) { return (int)(min(ek[0], ek[1]) >> 7); }

// inv = 1 / sqrt(mean + eps) of row xr (H <= 4096, H % 8 == 0, 16-byte
// aligned) with the mean from rms_mean_f: one wave; lane l sums the 16-byte
// chunks l, l + 64, ... (all loads issued at once), then wave reductions on
// the DPP path.
__device__ __forceinline__ float row_rms_inv(const uint16_t *__restrict__ xr, int H, float eps,
                                             int lane) {
  const int nch = H >> 3;
  u32x4 v[8];
#pragma unroll
  for (int c = 0; c < 8; ++c)
    v[c] = *(const u32x4 *)(xr + 8 * min(lane + 64 * c, nch - 1));
  double p4[4] = {0.0, 0.0, 0.0, 0.0};
  u16x2_t ek = {0x7F80, 0x7F80};
#pragma unroll
  for (int c = 0; c < 8; ++c)
    if (lane + 64 * c < nch) sumsq_chunk(v[c], p4, ek);
  const double tot = wave_sum_f64((p4[0] + p4[1]) + (p4[2] + p4[3]));
  const int emin = (int)wave_min_u32((uint32_t)ek_emin(ek));
  return rms_inv_finish(tot, emin, xr, H, eps, lane);
}

// two floats as packed bf16 (low half: lo), round to nearest even
// (v_cvt_pk_bf16_f32; for finite values the same bits as f32_to_bf16)
__device__ __forceinline__ uint32_t bf16x2_bits(float lo, float hi) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, bf16x2_t{(__bf16)lo, (__bf16)hi});
}

// one packed bf16 pair of x normalized as k_rmsnorm writes it: (x * inv) * wt
// in fp32, rounded to nearest even
__device__ __forceinline__ uint32_t norm_pair(uint32_t xp, uint32_t wp, float inv,
                                              const NormIn &n) {
  const float v0 = __uint_as_float(xp << 16) * inv, v1 = __uint_as_float(xp & 0xFFFF0000u) * inv;
  float w0 = 1.0f, w1 = 1.0f;
  if (n.w) {
    w0 = __uint_as_float(wp << 16);
    w1 = __uint_as_float(wp & 0xFFFF0000u);
    if (n.mode == AINFER_NORM_ONE_PLUS) {
      w0 = 1.0f + w0;
      w1 = 1.0f + w1;
    }
  }
  return bf16x2_bits(v0 * w0, v1 * w1);
}

// q8 / sq8 (optional): the row's W4A8 codes and group scales as well, the
// arithmetic of k_act_quant_i8 (ScalesMax + Quantize, kernels.cpp:551-579)
// on the values written (the 4 lanes holding a 128-wide group share its max)
__device__ __forceinline__ void write_xperm(const uint16_t *__restrict__ xrow,
                                            uint16_t *__restrict__ xperm,
                                            float *__restrict__ xsum, int t, int H, int lane,
                                            const NormIn *norm = nullptr, float inv = 1.0f,
                                            int8_t *__restrict__ q8 = nullptr,
                                            float *__restrict__ sq8 = nullptr) {
  {
    uint16_t *xo = xperm + (size_t)t * H;
    for (int b = lane; b < (H >> 5); b += 64) {
      const u32x4 *src = (const u32x4 *)(xrow + b * 32);
      const u32x4 s0 = src[0], s1 = src[1], s2 = src[2], s3 = src[3];
      uint32_t in[16] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3],
                         s2[0], s2[1], s2[2], s2[3], s3[0], s3[1], s3[2], s3[3]};
      if (norm && norm->on) {
        u32x4 wv[4] = {};
        if (norm->w) {
          const u32x4 *ws = (const u32x4 *)(norm->w + b * 32);
#pragma unroll
          for (int i = 0; i < 4; ++i) wv[i] = ws[i];
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) in[i] = norm_pair(in[i], wv[i >> 2][i & 3], inv, *norm);
      }
      uint32_t out[16];
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int e2 = 0; e2 < 4; ++e2) {
          const int ka = 8 * e2 + j, kb = ka + 4;
          const uint32_t lo = (in[ka >> 1] >> (16 * (ka & 1))) & 0xFFFFu;
          const uint32_t hi = (in[kb >> 1] >> (16 * (kb & 1))) & 0xFFFFu;
          out[4 * j + e2] = lo | (hi << 16);
        }
      u32x4 *dst = (u32x4 *)(xo + b * 32);
      dst[0] = u32x4{out[0], out[1], out[2], out[3]};
      dst[1] = u32x4{out[4], out[5], out[6], out[7]};
      dst[2] = u32x4{out[8], out[9], out[10], out[11]};
      dst[3] = u32x4{out[12], out[13], out[14], out[15]};
      if (xsum) {
        // sum of the 128-wide group: this block's 32 values, then the 4
        // consecutive lanes holding the group's blocks (fixed order)
        float bs = 0.0f;
#pragma unroll
        for (int i2 = 0; i2 < 16; ++i2)
          bs += __uint_as_float(in[i2] << 16) + __uint_as_float(in[i2] & 0xFFFF0000u);
        bs += __shfl_xor(bs, 1, 64);
        bs += __shfl_xor(bs, 2, 64);
        if ((b & 3) == 0) xsum[(size_t)t * (H >> 7) + (b >> 2)] = bs;
      }
      if (q8) {
        float m = 0.0f;  // the reference's running max from 0 (exact: any order)
#pragma unroll
        for (int i2 = 0; i2 < 16; ++i2) {
          const float a0 = fabsf(__uint_as_float(in[i2] << 16));
          const float a1 = fabsf(__uint_as_float(in[i2] & 0xFFFF0000u));
          m = a0 > m ? a0 : m;
          m = a1 > m ? a1 : m;
        }
        const float m1 = __shfl_xor(m, 1, 64);
        m = m1 > m ? m1 : m;
        const float m2 = __shfl_xor(m, 2, 64);
        m = m2 > m ? m2 : m;
        float sc = m / 127.0f;
        sc = sc == 0.0f ? 1.0f : sc;
        uint32_t pk[8];
#pragma unroll
        for (int i2 = 0; i2 < 8; ++i2) pk[i2] = 0u;
#pragma unroll
        for (int i2 = 0; i2 < 32; ++i2) {
          const uint32_t w = in[i2 >> 1];
          const float v = __uint_as_float((i2 & 1) ? (w & 0xFFFF0000u) : (w << 16));
          const float r = v / sc;
          int qi = (int)(r >= 0.0f ? r + 0.5f : r - 0.5f);
          qi = qi < -127 ? -127 : (qi > 127 ? 127 : qi);
          pk[i2 >> 2] |= (uint32_t)(uint8_t)qi << (8 * (i2 & 3));
        }
        u32x4 *qd = (u32x4 *)(q8 + (size_t)t * H + b * 32);
        qd[0] = u32x4{pk[0], pk[1], pk[2], pk[3]};
        qd[1] = u32x4{pk[4], pk[5], pk[6], pk[7]};
        if ((b & 3) == 0) sq8[(size_t)t * (H >> 7) + (b >> 2)] = sc;
      }
    }
  }
}
