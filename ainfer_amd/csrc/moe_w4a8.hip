// moe_w4a8.hip - the reference's production GEMV numerics (W4A8) on gfx950:
// per-group-128 int8 activation quantisation and the INT4 x int8 GEMV.
//
// Reference arithmetic (restated, not translated):
//  - ScalesMax + Quantize (tools/cmdlist/kernels.cpp:551-579): per group of
//    128, SQ = max|x| / 127 (0 -> 1), q = trunc(x/SQ +- 0.5) clamped to
//    [-127, 127];
//  - Int4Gemv (tools/cmdlist/kernels.cpp:148-201): per row m,
//    y = sum over groups g in order of float(gs) * s_w[m][g] * SQ[g], with
//    gs the exact int32 dot of the group's nibbles and int8 activations.
//
// gfx950 form: a block owns 16 rows x 16 tokens, its waves split the
// groups.  One group is one 16-byte load per lane (row l%16, k-quarter l/16)
// and two v_mfma_i32_16x16x64_i8: the nibbles' even and odd halves, each
// widened to bytes q+8 in [0, 15] by one xor and one and.  The activation
// bytes are permuted with v_perm_b32 into the same k order, so A and B agree
// on every k.  gs = D(q+8) - 8 * D(ones), exact in int32; each group's term
// float(gs) * s * sq is rounded as the reference rounds it, and the terms
// are added in group order with no contraction, so each y is bit-identical
// to the reference formula.
#include <type_traits>

#include "moe_common.h"
#include "moe_internal.h"

namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));

// one wave per (token, group of 128): two elements per lane.
// A second row set (x2, T2, K2 -> q2, sq2) takes the items past T * K / 128,
// so two quantizations share a launch.
template <typename XT>
__global__ __launch_bounds__(256) void k_act_quant_i8(const XT *__restrict__ x, int T, int K,
                                                      int8_t *__restrict__ q,
                                                      float *__restrict__ sq,
                                                      const XT *__restrict__ x2 = nullptr,
                                                      int T2 = 0, int K2 = 128,
                                                      int8_t *__restrict__ q2 = nullptr,
                                                      float *__restrict__ sq2 = nullptr) {
  int item = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (item >= T * (K / 128)) {
    item -= T * (K / 128);
    if (item >= T2 * (K2 / 128)) return;
    x = x2;
    T = T2;
    K = K2;
    q = q2;
    sq = sq2;
  }
  const int G = K / 128;
  const int t = item / G, g = item % G;
  const size_t base = (size_t)t * K + (size_t)g * 128 + 2 * lane;
  float v[2];
  if constexpr (sizeof(XT) == 4) {
    const float2 p = *(const float2 *)(x + base);
    v[0] = p.x;
    v[1] = p.y;
  } else {
    const uint32_t p = *(const uint32_t *)(x + base);
    v[0] = __uint_as_float(p << 16);
    v[1] = __uint_as_float(p & 0xFFFF0000u);
  }
  // the reference's running max (a > m ? a : m from 0, so NaNs drop out);
  // max is exact, so the lane-tree order does not matter
  float m = 0.0f;
  for (int i = 0; i < 2; ++i) {
    const float a = fabsf(v[i]);
    m = a > m ? a : m;
  }
  m = __uint_as_float(wave_max_u32(__float_as_uint(m)));
  float s = m / 127.0f;
  s = s == 0.0f ? 1.0f : s;
  int8_t out[2];
  for (int i = 0; i < 2; ++i) {
    const float r = v[i] / s;
    int qi = (int)(r >= 0.0f ? r + 0.5f : r - 0.5f);
    qi = qi < -127 ? -127 : (qi > 127 ? 127 : qi);
    out[i] = (int8_t)qi;
  }
  *(uint16_t *)(q + base) = (uint16_t)((uint8_t)out[0] | ((uint16_t)(uint8_t)out[1] << 8));
  if (lane == 0) sq[(size_t)t * G + g] = s;
}

__device__ __forceinline__ i32x4 mfma_i8(i32x4 a, i32x4 b, i32x4 c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

#ifndef GV_WAVES
#define GV_WAVES 4  // waves per GEMV block, split over the groups
#endif
#ifndef GV_GPW
#define GV_GPW 2  // groups per wave per pass, loads issued together
#endif
constexpr int GV_CHUNK = GV_WAVES * GV_GPW;  // groups whose terms one LDS pass holds
static_assert(GV_WAVES >= 4, "the ordered sum uses one thread per (row, token) of a 16 x 16 tile");

// One 16-row x 16-token block of the INT4 x int8 GEMV, GV_WAVES waves: rows
// [m0, +16) of P / S (M rows, K columns) against 16 activation rows, lane
// column c reading row xrow of xq / sq.  Wave w computes the terms
// float(gs) * s * sq of groups w, w + GV_WAVES, ... of each chunk into LDS;
// then 256 threads, one per (row, token), add them in group order.  Returns
// the sum of thread (row 4 * (lp / 16) + i, token lp % 16), lp = tid / 4,
// i = tid % 4.
// STG: the block's weight scales [16][G] and activation scales [16][G] are
// staged in LDS (gv_lds) once (per-lane 2-byte gathers in every pass cost 3
// of 18 us at 17408 x 5120); else they are gathered per group.
template <int SD, bool STG>
__device__ __forceinline__ float gemv_i8_block(const uint8_t *__restrict__ P,
                                               const uint16_t *__restrict__ S, int m0, int M,
                                               int K, const int8_t *__restrict__ xq,
                                               const float *__restrict__ sq, int xrow,
                                               float (*term)[256], uint8_t *gv_lds,
                                               const int *xrows_lds) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int G = K / 128, qd = lane >> 4, c = lane & 15;
  // A operand: row m0 + c; B operand and D column: token column c
  const uint8_t *wp = P + (size_t)min(m0 + c, M - 1) * (K / 2) + qd * 16;
  const int8_t *xp = xq + (size_t)xrow * K + qd * 32;
  const float *sqp = sq + (size_t)xrow * G;
  // D rows of this lane: m0 + 4 * qd + i
  const uint16_t *sp[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) sp[i] = S + (size_t)min(m0 + 4 * qd + i, M - 1) * G;
  float *sq_l = (float *)gv_lds;
  uint16_t *sc_l = (uint16_t *)(gv_lds + 16 * G * 4);
  if constexpr (STG) {
    for (int i = threadIdx.x; i < 16 * G; i += GV_WAVES * 64) {
      const int r = i / G, g = i - r * G;
      sc_l[i] = S[(size_t)min(m0 + r, M - 1) * G + g];
      sq_l[i] = sq[(size_t)xrows_lds[r] * G + g];
    }
    __syncthreads();
  }
  const i32x4 ones = {0x01010101, 0x01010101, 0x01010101, 0x01010101};
  const i32x4 zero = {0, 0, 0, 0};
  float acc = 0.0f;
  for (int c0 = 0; c0 < G; c0 += GV_CHUNK) {
    const int cn = min(GV_CHUNK, G - c0);
    // every load of the pass first (clamped to the last group; the terms
    // past the chunk are not stored)
    u32x4 wv[GV_GPW], xav[GV_GPW], xbv[GV_GPW];
    uint16_t scv[GV_GPW][4];
    float sqv[GV_GPW];
#pragma unroll
    for (int jj = 0; jj < GV_GPW; ++jj) {
      const int g = c0 + min(wave + jj * GV_WAVES, cn - 1);
      wv[jj] = __builtin_nontemporal_load((const u32x4 *)(wp + (size_t)g * 64));
      xav[jj] = *(const u32x4 *)(xp + (size_t)g * 128);
      xbv[jj] = *(const u32x4 *)(xp + (size_t)g * 128 + 16);
      if constexpr (!STG) {
#pragma unroll
        for (int i = 0; i < 4; ++i) scv[jj][i] = sp[i][g];
        sqv[jj] = sqp[g];
      }
    }
#pragma unroll
    for (int jj = 0; jj < GV_GPW; ++jj) {
      const int j = wave + jj * GV_WAVES;
      const u32x4 w = wv[jj], xa = xav[jj], xb = xbv[jj];
      float sc[4];
      float sqg;
      if constexpr (STG) {
        const int g = c0 + min(j, cn - 1);
#pragma unroll
        for (int i = 0; i < 4; ++i) sc[i] = scale_to_f32<SD>(sc_l[(4 * qd + i) * G + g]);
        sqg = sq_l[c * G + g];
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) sc[i] = scale_to_f32<SD>(scv[jj][i]);
        sqg = sqv[jj];
      }
      i32x4 a0, a1, b0, b1;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const uint32_t u = w[jj] ^ 0x88888888u;  // nibble q -> q + 8
        a0[jj] = (int)(u & 0x0F0F0F0Fu);         // k = 8jj + {0, 2, 4, 6}
        a1[jj] = (int)((u >> 4) & 0x0F0F0F0Fu);  // k = 8jj + {1, 3, 5, 7}
      }
      b0[0] = (int)__builtin_amdgcn_perm(xa[1], xa[0], 0x06040200u);
      b0[1] = (int)__builtin_amdgcn_perm(xa[3], xa[2], 0x06040200u);
      b0[2] = (int)__builtin_amdgcn_perm(xb[1], xb[0], 0x06040200u);
      b0[3] = (int)__builtin_amdgcn_perm(xb[3], xb[2], 0x06040200u);
      b1[0] = (int)__builtin_amdgcn_perm(xa[1], xa[0], 0x07050301u);
      b1[1] = (int)__builtin_amdgcn_perm(xa[3], xa[2], 0x07050301u);
      b1[2] = (int)__builtin_amdgcn_perm(xb[1], xb[0], 0x07050301u);
      b1[3] = (int)__builtin_amdgcn_perm(xb[3], xb[2], 0x07050301u);
      i32x4 d = mfma_i8(a0, b0, zero);
      d = mfma_i8(a1, b1, d);
      i32x4 sx = mfma_i8(ones, b0, zero);
      sx = mfma_i8(ones, b1, sx);
      f32x4 tv;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma clang fp contract(off)
        const int gs = d[i] - 8 * sx[i];
        tv[i] = (float)gs * sc[i] * sqg;  // the reference's product, unfused
      }
      if (j < cn) *(f32x4 *)&term[j][lane * 4] = tv;
    }
    __syncthreads();
    {
#pragma clang fp contract(off)
      for (int j = 0; j < cn; ++j) acc = acc + term[j][threadIdx.x];  // group order
    }
    __syncthreads();
  }
  return acc;
}

// grid (ceil(M / 16), ceil(T / 16)): the block owns rows [16 * bx, +16) and
// tokens [16 * by, +16).  y is [T][M] fp32.
template <int SD, bool STG>
__global__ __launch_bounds__(GV_WAVES * 64) void k_int4_gemv_i8(
    const uint8_t *__restrict__ P, const uint16_t *__restrict__ S, const int8_t *__restrict__ xq,
    const float *__restrict__ sq, int M, int K, int T, float *__restrict__ y) {
  __shared__ float term[GV_CHUNK][256];
  __shared__ int xrows[16];
  extern __shared__ __attribute__((aligned(16))) uint8_t gv_lds[];  // STG: [16][G] f32, [16][G] u16
  const int m0 = blockIdx.x * 16, t0 = blockIdx.y * 16;
  if (threadIdx.x < 16) xrows[threadIdx.x] = min(t0 + (int)threadIdx.x, T - 1);
  __syncthreads();
  const int c = threadIdx.x & 15;
  const float acc = gemv_i8_block<SD, STG>(P, S, m0, M, K, xq, sq, min(t0 + c, T - 1), term,
                                           gv_lds, xrows);
  // element e = lane' * 4 + i of the producing lane': row 4 * (lane' / 16) + i,
  // token lane' % 16
  const int lp = threadIdx.x >> 2, i = threadIdx.x & 3;
  const int m = m0 + 4 * (lp >> 4) + i, t = t0 + (lp & 15);
  if (m < M && t < T) y[(size_t)t * M + m] = acc;
}

// ---- T = 1: the GEMV proper -------------------------------------------------
// One token, so no MFMA: a wave owns GV1_RW consecutive rows, lane l the
// 16-byte chunks l, l + 64, ... of each (one load instruction = 1 KB of one
// row, the wide pattern that streams fastest).  Chunk c is quarter c % 4 of
// group c / 4, so the four lanes of a quad hold one group: the exact int32
// dot of its nibbles and int8 activations is four v_dot4_i32_i8 per lane
// (q + 8 in [0, 15] against x, less 8 * sum(x)) and a quad sum.  The terms
// float(gs) * s * sq go to LDS and lane r adds row r's in group order.
#ifndef GV1_RW
#define GV1_RW 2  // rows per wave (2: 10.0 us at 17408 x 5120; 1: 12.1, 4: 10.9, 8: 13.0)
#endif
#ifndef GV1_WAVES
#define GV1_WAVES 4  // waves per block (4: 10.0-10.3 us at 17408 x 5120; 2: 10.0, 8: 10.6, 16: 12.9)
#endif

// Rows [m0, m0 + GV1_RW) of NMAT matrices P[j] / S[j] (M rows, K columns)
// against one activation row xq / sq.  Lane j * GV1_RW + r returns row
// m0 + r of matrix j (other lanes 0).  term: this wave's LDS, NMAT * GV1_RW
// rows of NC * 16 floats.  Every weight load of every matrix is issued
// before any is used.
struct NoHook {
  __device__ void operator()() const {}
};
template <int SD, int NC, int NMAT, typename Hook = NoHook>
__device__ __forceinline__ float gemv1_rows(const uint8_t *const (&P)[NMAT],
                                            const uint16_t *const (&S)[NMAT], int m0, int M,
                                            int K, const int8_t *xq, const float *sq,
                                            float *term, int lane, Hook hook = Hook()) {
  constexpr int R = NMAT * GV1_RW;
  const int C = K >> 5, G = K >> 7;  // 16-byte chunks and groups per row
  const size_t rowb = (size_t)K / 2;
  u32x4 wv[R][NC];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const uint8_t *wp = P[r / GV1_RW] + (size_t)min(m0 + r % GV1_RW, M - 1) * rowb;
#pragma unroll
    for (int i = 0; i < NC; ++i)
      wv[r][i] = __builtin_nontemporal_load((const u32x4 *)(wp + (size_t)min(lane + 64 * i, C - 1) * 16));
  }
  // with the weights in flight: whatever produces xq / sq (the block's
  // quantization of its activation row into LDS)
  hook();
  // activations of this lane's chunks (32 bytes each, the same for every
  // row), the group scales of its quad's groups, and the weight scales
  u32x4 xa[NC], xb[NC];
  float sqv[NC];
  uint16_t sc[R][NC];
  const int qg = lane >> 2;  // group of chunk lane + 64 i is qg + 16 i
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int ch = min(lane + 64 * i, C - 1), g = min(qg + 16 * i, G - 1);
    xa[i] = *(const u32x4 *)(xq + (size_t)ch * 32);
    xb[i] = *(const u32x4 *)(xq + (size_t)ch * 32 + 16);
    sqv[i] = sq[g];
#pragma unroll
    for (int r = 0; r < R; ++r)
      sc[r][i] = S[r / GV1_RW][(size_t)min(m0 + r % GV1_RW, M - 1) * G + g];
  }
  // x in the nibbles' order: the low nibbles of weight dword d are elements
  // 8 d + {0, 2, 4, 6}, the high ones 8 d + {1, 3, 5, 7}
  int xe[NC][4], xo[NC][4], sx[NC];
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const uint32_t b[8] = {xa[i][0], xa[i][1], xa[i][2], xa[i][3],
                           xb[i][0], xb[i][1], xb[i][2], xb[i][3]};
    int s = 0;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      xe[i][d] = (int)__builtin_amdgcn_perm(b[2 * d + 1], b[2 * d], 0x06040200u);
      xo[i][d] = (int)__builtin_amdgcn_perm(b[2 * d + 1], b[2 * d], 0x07050301u);
      s = __builtin_amdgcn_sdot4(xe[i][d], 0x01010101, s, false);
      s = __builtin_amdgcn_sdot4(xo[i][d], 0x01010101, s, false);
    }
    sx[i] = 8 * s;
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      int d = -sx[i];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t u = wv[r][i][j] ^ 0x88888888u;  // nibble q -> q + 8
        d = __builtin_amdgcn_sdot4((int)(u & 0x0F0F0F0Fu), xe[i][j], d, false);
        d = __builtin_amdgcn_sdot4((int)((u >> 4) & 0x0F0F0F0Fu), xo[i][j], d, false);
      }
      if (lane + 64 * i >= C) d = 0;
      d += __builtin_amdgcn_mov_dpp(d, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
      d += __builtin_amdgcn_mov_dpp(d, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
      const int g = qg + 16 * i;
      if ((lane & 3) == 0 && g < G) {
#pragma clang fp contract(off)
        term[r * NC * 16 + g] = (float)d * scale_to_f32<SD>(sc[r][i]) * sqv[i];  // unfused
      }
    }
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  float acc = 0.0f;
  if (lane < R) {
#pragma clang fp contract(off)
    for (int g = 0; g < G; ++g) acc = acc + term[lane * NC * 16 + g];  // group order
  }
  return acc;
}

template <int SD, int NC>
__global__ __launch_bounds__(GV1_WAVES * 64) void k_int4_gemv_i8_t1(
    const uint8_t *__restrict__ P, const uint16_t *__restrict__ S, const int8_t *__restrict__ xq,
    const float *__restrict__ sq, int M, int K, float *__restrict__ y) {
  __shared__ float term[GV1_WAVES][GV1_RW * NC * 16];
  const int tx = tid_opaque();
  const int wave = __builtin_amdgcn_readfirstlane(tx >> 6), lane = tx & 63;
  const int m0 = (blockIdx.x * GV1_WAVES + wave) * GV1_RW;
  const uint8_t *const Pm[1] = {P};
  const uint16_t *const Sm[1] = {S};
  const float acc = gemv1_rows<SD, NC, 1>(Pm, Sm, m0, M, K, xq, sq, term[wave], lane);
  if (lane < GV1_RW && m0 + lane < M) y[m0 + lane] = acc;
}

// One fp32 row x[0, K) quantized per group of 128 into LDS by a whole block
// of GV1_WAVES waves, the arithmetic of k_act_quant_i8 (ScalesMax + Quantize,
// tools/cmdlist/kernels.cpp:551-579): thread l takes elements 1024 j + 4 l +
// [0, 4), so each half-wave covers one group and its max is a 32-lane
// reduction (max is exact: the order does not matter).  K <= 4096.  The
// loads (quant_row_load) are issued before the weight loads, so the
// quantization (quant_row_lds) waits for them alone.
struct QRow {
  float4 v[4];
};
__device__ __forceinline__ QRow quant_row_load(const float *__restrict__ x, int K) {
  static_assert(GV1_WAVES == 4, "a block of 256 threads covers 1024 elements per step");
  QRow r;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = 1024 * j + 4 * (int)threadIdx.x;
    r.v[j] = e < K ? *(const float4 *)(x + e) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  return r;
}
__device__ __forceinline__ void quant_row_lds(const QRow &r, int K, int8_t *q, float *sq) {
  const int lid = threadIdx.x;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = 1024 * j + 4 * lid;
    if (1024 * j >= K) break;
    const float vv[4] = {r.v[j].x, r.v[j].y, r.v[j].z, r.v[j].w};
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float a = fabsf(vv[i]);
      m = a > m ? a : m;
    }
#pragma unroll
    for (int o = 16; o >= 1; o >>= 1)
      m = __uint_as_float(max(__float_as_uint(m), (uint32_t)__shfl_xor((int)__float_as_uint(m), o, 64)));
    float sc = m / 127.0f;
    sc = sc == 0.0f ? 1.0f : sc;
    uint32_t packed = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float rr = vv[i] / sc;
      int qi = (int)(rr >= 0.0f ? rr + 0.5f : rr - 0.5f);
      qi = qi < -127 ? -127 : (qi > 127 ? 127 : qi);
      packed |= (uint32_t)(uint8_t)(int8_t)qi << (8 * i);
    }
    if (e < K) {
      *(uint32_t *)(q + e) = packed;
      if ((lid & 31) == 0) sq[e >> 7] = sc;
    }
  }
}

// The layer's expert GEMVs at T = 1 (every dispatch tile holds one token):
// grid (ceil(N / (GV1_WAVES * GV1_RW)), tiles), the rows of gemv1_rows.
//   MODE 0: act[pos][n] = silu(gate . x) * (up . x), fp32 (SiluMul,
//           tools/cmdlist/kernels.cpp:29-37);
//   MODE 1: o[pos][h] = down . act.
template <int SD, int MODE, int NC, bool QIN = false>
__global__ __launch_bounds__(GV1_WAVES * 64) void k_w4a8_expert_t1(W4A8Args a) {
  constexpr int NMAT = MODE == 0 ? 2 : 1;
  __shared__ float term[GV1_WAVES][NMAT * GV1_RW * NC * 16];
  // QIN: the block's own int8 copy of its fp32 activation row
  __shared__ __attribute__((aligned(16))) int8_t q_l[QIN ? 4096 : 16];
  __shared__ float sq_l[QIN ? 32 : 1];
  if ((int)blockIdx.y >= *a.n_tiles) return;
  const int4 t = a.tiles[blockIdx.y];
  const int e = t.x, pos0 = t.y;
  const bool shared = e == a.E;
  const int N = MODE == 0 ? (shared ? a.Is : a.I) : a.H;
  const int K = MODE == 0 ? a.H : (shared ? a.Is : a.I);
  const int tx = tid_opaque();
  const int wave = __builtin_amdgcn_readfirstlane(tx >> 6), lane = tx & 63;
  const int m0 = (blockIdx.x * GV1_WAVES + wave) * GV1_RW;
  // (QIN: every wave of the block takes part in the quantization; the host
  // keeps N a multiple of the block's rows there)
  if (!QIN && m0 >= N) return;
  const size_t rowb = (size_t)K / 2, G = K / 128;
  if constexpr (MODE == 0) {
    const int tok = shared ? pos0 : a.ptok[pos0];
    const uint8_t *const Pm[2] = {shared ? a.ws0 : a.w0 + (size_t)e * N * rowb,
                                  shared ? a.ws1 : a.w1 + (size_t)e * N * rowb};
    const uint16_t *const Sm[2] = {shared ? a.ss0 : a.s0 + (size_t)e * N * G,
                                   shared ? a.ss1 : a.s1 + (size_t)e * N * G};
    const float v = gemv1_rows<SD, NC, 2>(Pm, Sm, m0, N, K, a.xq + (size_t)tok * K,
                                          a.xs + (size_t)tok * G, term[wave], lane);
    // lane r: gate row m0 + r; lane GV1_RW + r: up row m0 + r
    const float u = __shfl(v, lane + GV1_RW, 64);
    if (lane < GV1_RW && m0 + lane < N)
      (shared ? a.act_s : a.act)[(size_t)pos0 * N + m0 + lane] = v / (1.0f + expf(-v)) * u;
  } else {
    const uint8_t *const Pm[1] = {shared ? a.ws0 : a.w0 + (size_t)e * N * rowb};
    const uint16_t *const Sm[1] = {shared ? a.ss0 : a.s0 + (size_t)e * N * G};
    float v;
    if constexpr (QIN) {
      const QRow xr = quant_row_load((shared ? a.act_s : a.act) + (size_t)pos0 * K, K);
      v = gemv1_rows<SD, NC, 1>(Pm, Sm, m0, N, K, q_l, sq_l, term[wave], lane, [&]() {
        quant_row_lds(xr, K, q_l, sq_l);
        __syncthreads();
      });
    } else {
      const int8_t *aq = (shared ? a.aq_s : a.aq) + (size_t)pos0 * K;
      const float *as = (shared ? a.as_s : a.as) + (size_t)pos0 * G;
      v = gemv1_rows<SD, NC, 1>(Pm, Sm, m0, N, K, aq, as, term[wave], lane);
    }
    if (lane < GV1_RW && m0 + lane < N)
      a.o[(size_t)((shared ? a.T * a.k : 0) + pos0) * N + m0 + lane] = v;
  }
}

// ---- the MoE layer in W4A8 (AINFER_PRECISION_W4A8) --------------------------
// The decoder MLP of tools/decode/decode_l0.cpp:663-674 per (token, expert):
// xq -> Int4Gemv gate, Int4Gemv up -> SiluMul -> quantize -> Int4Gemv down,
// here grouped by expert: one block = 16 weight rows x one dispatch tile of
// at most 16 tokens of one expert (the shared expert's tiles carry expert id
// E), the GEMV block arithmetic above.
//   MODE 0: act[pos][n] = silu(gate . x) * (up . x), fp32, for the tile's
//           tokens (x quantized per 128-group, rows xq[token]);
//   MODE 1: o[pos][h] = down . act, fp32, act quantized per 128-group
//           (rows actq[pos]; the shared expert's outputs at rows T * k + t).
template <int SD, int MODE>
__global__ __launch_bounds__(GV_WAVES * 64) void k_w4a8_expert(W4A8Args a) {
  __shared__ float term[GV_CHUNK][256];
  __shared__ int xrows[16];
  extern __shared__ __attribute__((aligned(16))) uint8_t gv_lds[];
  if ((int)blockIdx.y >= *a.n_tiles) return;
  const int4 t = a.tiles[blockIdx.y];
  const int e = t.x, pos0 = t.y, mcnt = t.z;
  const bool shared = e == a.E;
  const int N = MODE == 0 ? (shared ? a.Is : a.I) : a.H;
  const int K = MODE == 0 ? a.H : (shared ? a.Is : a.I);
  const int m0 = blockIdx.x * 16;
  if (m0 >= N) return;
  // the tile's activation rows (columns past mcnt repeat the last one)
  if (threadIdx.x < 16) {
    const int r = min((int)threadIdx.x, mcnt - 1);
    xrows[threadIdx.x] = MODE == 0 ? (shared ? pos0 + r : a.ptok[pos0 + r]) : pos0 + r;
  }
  __syncthreads();
  const int c = threadIdx.x & 15;
  const int xr = xrows[c];
  const size_t rowb = (size_t)K / 2, G = K / 128;
  float v;
  if constexpr (MODE == 0) {
    const uint8_t *wg = shared ? a.ws0 : a.w0 + (size_t)e * N * rowb;
    const uint8_t *wu = shared ? a.ws1 : a.w1 + (size_t)e * N * rowb;
    const uint16_t *sgp = shared ? a.ss0 : a.s0 + (size_t)e * N * G;
    const uint16_t *sup = shared ? a.ss1 : a.s1 + (size_t)e * N * G;
    const float g = gemv_i8_block<SD, true>(wg, sgp, m0, N, K, a.xq, a.xs, xr, term, gv_lds, xrows);
    const float u = gemv_i8_block<SD, true>(wu, sup, m0, N, K, a.xq, a.xs, xr, term, gv_lds, xrows);
    v = g / (1.0f + expf(-g)) * u;  // SiluMul, tools/cmdlist/kernels.cpp:29-37
  } else {
    const uint8_t *wd = shared ? a.ws0 : a.w0 + (size_t)e * N * rowb;
    const uint16_t *sdp = shared ? a.ss0 : a.s0 + (size_t)e * N * G;
    v = gemv_i8_block<SD, true>(wd, sdp, m0, N, K, shared ? a.aq_s : a.aq,
                                shared ? a.as_s : a.as, xr, term, gv_lds, xrows);
  }
  const int lp = threadIdx.x >> 2, i = threadIdx.x & 3;
  const int m = m0 + 4 * (lp >> 4) + i, tc = lp & 15;
  if (m >= N || tc >= mcnt) return;
  if constexpr (MODE == 0)
    (shared ? a.act_s : a.act)[(size_t)(pos0 + tc) * N + m] = v;
  else
    a.o[(size_t)((shared ? a.T * a.k : 0) + pos0 + tc) * N + m] = v;
}

// y[t][h] = bf16(sum_j w_j o[pos(t, j)][h] + g_s o[T * k + t][h] (+ resid)),
// fp32 fma in slot order (k_combine's order on the fp32 expert outputs).
__global__ __launch_bounds__(256) void k_combine_f32(const float *__restrict__ o,
                                                     const int32_t *__restrict__ inv,
                                                     const float *__restrict__ w,
                                                     const float *__restrict__ sg,
                                                     int has_shared,
                                                     const uint16_t *__restrict__ resid,
                                                     uint16_t *__restrict__ y, int T, int k, int H,
                                                     const int32_t *__restrict__ err) {
  const int t = blockIdx.y, h = blockIdx.x * 256 + threadIdx.x;
  if (h >= H) return;
  float acc = 0.0f;
  for (int j = 0; j < k; ++j)
    acc = __builtin_fmaf(w[(size_t)t * k + j], o[(size_t)inv[(size_t)t * k + j] * H + h], acc);
  if (has_shared) acc = __builtin_fmaf(sg[t], o[((size_t)T * k + t) * H + h], acc);
  if (resid) acc += bf16_to_f32(resid[(size_t)t * H + h]);
  y[(size_t)t * H + h] = (err && *err) ? (uint16_t)0x7FC0u : f32_to_bf16(acc);
}

}  // namespace

hipError_t launch_act_quant_i8(const void *x, int x_dtype, int T, int K, int8_t *q, float *sq,
                               hipStream_t s) {
  const int items = T * (K / 128);
  const unsigned grid = (items + 3) / 4;
  if (x_dtype == AINFER_ACT_F32)
    k_act_quant_i8<float><<<grid, 256, 0, s>>>((const float *)x, T, K, q, sq);
  else
    k_act_quant_i8<uint16_t><<<grid, 256, 0, s>>>((const uint16_t *)x, T, K, q, sq);
  return hipGetLastError();
}

hipError_t launch_act_quant_f32_pair(const float *x, int T, int K, int8_t *q, float *sq,
                                     const float *x2, int T2, int K2, int8_t *q2, float *sq2,
                                     hipStream_t s) {
  const int items = T * (K / 128) + (x2 ? T2 * (K2 / 128) : 0);
  if (items == 0) return hipSuccess;
  k_act_quant_i8<float><<<(items + 3) / 4, 256, 0, s>>>(x, T, K, q, sq, x2, x2 ? T2 : 0,
                                                        x2 ? K2 : 128, q2, sq2);
  return hipGetLastError();
}

hipError_t launch_w4a8_expert(int mode, int scale_dtype, const W4A8Args &a, int max_tiles,
                              hipStream_t s) {
  if (max_tiles <= 0) return hipSuccess;
  const int N = mode == 0 ? (a.I > a.Is ? a.I : a.Is) : a.H;
  const int K = mode == 0 ? a.H : (a.I > a.Is ? a.I : a.Is);
  const int Kmin = mode == 0 ? a.H : (a.Is > 0 && a.Is < a.I ? a.Is : a.I);
  if (a.T == 1 && K <= 8192 && Kmin % 128 == 0) {
    // one token per tile: the wide one-token rows (gemv1_rows)
    const int nc = (K / 32 + 63) / 64;
    const dim3 g1((N + GV1_WAVES * GV1_RW - 1) / (GV1_WAVES * GV1_RW), max_tiles);
    // the in-kernel quantization needs whole blocks of rows and K <= 4096
    const bool qin = mode == 1 && a.quant_in && a.H % (GV1_WAVES * GV1_RW) == 0 && K <= 4096;
    if (mode == 1 && a.quant_in && !qin) {
      hipError_t e = launch_act_quant_f32_pair(a.act, a.T * a.k, a.I, const_cast<int8_t *>(a.aq),
                                               const_cast<float *>(a.as), a.Is > 0 ? a.act_s : nullptr,
                                               a.T, a.Is, const_cast<int8_t *>(a.aq_s),
                                               const_cast<float *>(a.as_s), s);
      if (e != hipSuccess) return e;
    }
    auto go1 = [&](auto sd_c, auto nc_c) {
      constexpr int SDc = decltype(sd_c)::value, NCc = decltype(nc_c)::value;
      if (mode == 0)
        k_w4a8_expert_t1<SDc, 0, NCc><<<g1, GV1_WAVES * 64, 0, s>>>(a);
      else if (qin)
        k_w4a8_expert_t1<SDc, 1, NCc, true><<<g1, GV1_WAVES * 64, 0, s>>>(a);
      else
        k_w4a8_expert_t1<SDc, 1, NCc><<<g1, GV1_WAVES * 64, 0, s>>>(a);
    };
    auto go_nc = [&](auto sd_c) {
      if (nc == 1) go1(sd_c, std::integral_constant<int, 1>());
      else if (nc == 2) go1(sd_c, std::integral_constant<int, 2>());
      else if (nc == 3) go1(sd_c, std::integral_constant<int, 3>());
      else go1(sd_c, std::integral_constant<int, 4>());
    };
    if (scale_dtype == AINFER_SCALE_FP16)
      go_nc(std::integral_constant<int, AINFER_SCALE_FP16>());
    else
      go_nc(std::integral_constant<int, AINFER_SCALE_BF16>());
    return hipGetLastError();
  }
  if (mode == 1 && a.quant_in) {
    hipError_t e = launch_act_quant_f32_pair(a.act, a.T * a.k, a.I, const_cast<int8_t *>(a.aq),
                                             const_cast<float *>(a.as), a.Is > 0 ? a.act_s : nullptr,
                                             a.T, a.Is, const_cast<int8_t *>(a.aq_s),
                                             const_cast<float *>(a.as_s), s);
    if (e != hipSuccess) return e;
  }
  const dim3 grid((N + 15) / 16, max_tiles);
  const size_t stg = (size_t)16 * (K / 128) * 6;  // staged scales
  auto go = [&](auto sd_c) {
    constexpr int SDc = decltype(sd_c)::value;
    if (mode == 0)
      k_w4a8_expert<SDc, 0><<<grid, GV_WAVES * 64, stg, s>>>(a);
    else
      k_w4a8_expert<SDc, 1><<<grid, GV_WAVES * 64, stg, s>>>(a);
  };
  if (scale_dtype == AINFER_SCALE_FP16)
    go(std::integral_constant<int, AINFER_SCALE_FP16>());
  else
    go(std::integral_constant<int, AINFER_SCALE_BF16>());
  return hipGetLastError();
}

hipError_t launch_combine_f32(const float *o, const int32_t *inv, const float *w,
                              const float *sg, int has_shared, const void *resid, void *y, int T,
                              int k, int H, const int32_t *err, hipStream_t s) {
  if (T == 0) return hipSuccess;
  k_combine_f32<<<dim3((H + 255) / 256, T), 256, 0, s>>>(
      o, inv, w, sg, has_shared, (const uint16_t *)resid, (uint16_t *)y, T, k, H, err);
  return hipGetLastError();
}

hipError_t launch_int4_gemv_i8(const uint8_t *P, const void *S, int scale_dtype, const int8_t *xq,
                               const float *sq, int M, int K, int T, float *y, hipStream_t s) {
  if (T == 1 && K % 128 == 0 && K <= 8192) {
    const int nc = (K / 32 + 63) / 64;
    const unsigned g1 = (unsigned)((M + GV1_WAVES * GV1_RW - 1) / (GV1_WAVES * GV1_RW));
    auto go1 = [&](auto sd_c, auto nc_c) {
      k_int4_gemv_i8_t1<decltype(sd_c)::value, decltype(nc_c)::value>
          <<<g1, GV1_WAVES * 64, 0, s>>>(P, (const uint16_t *)S, xq, sq, M, K, y);
    };
    auto go_nc = [&](auto sd_c) {
      if (nc == 1) go1(sd_c, std::integral_constant<int, 1>());
      else if (nc == 2) go1(sd_c, std::integral_constant<int, 2>());
      else if (nc == 3) go1(sd_c, std::integral_constant<int, 3>());
      else go1(sd_c, std::integral_constant<int, 4>());
    };
    if (scale_dtype == AINFER_SCALE_FP16)
      go_nc(std::integral_constant<int, AINFER_SCALE_FP16>());
    else
      go_nc(std::integral_constant<int, AINFER_SCALE_BF16>());
    return hipGetLastError();
  }
  const dim3 grid((M + 15) / 16, (T + 15) / 16);
  const size_t stg = (size_t)16 * (K / 128) * 6;  // staged scales
  const bool st = stg <= 48 * 1024;
  auto go = [&](auto sd_c, auto stg_c) {
    constexpr int SDc = decltype(sd_c)::value;
    constexpr bool STc = decltype(stg_c)::value;
    k_int4_gemv_i8<SDc, STc><<<grid, GV_WAVES * 64, STc ? stg : 0, s>>>(
        P, (const uint16_t *)S, xq, sq, M, K, T, y);
  };
  using F16 = std::integral_constant<int, AINFER_SCALE_FP16>;
  using B16 = std::integral_constant<int, AINFER_SCALE_BF16>;
  if (scale_dtype == AINFER_SCALE_FP16) {
    if (st) go(F16(), std::true_type()); else go(F16(), std::false_type());
  } else {
    if (st) go(B16(), std::true_type()); else go(B16(), std::false_type());
  }
  return hipGetLastError();
}
