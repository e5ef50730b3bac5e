// moe_expert.hip - grouped INT4 expert kernels, small-M form (decode).
//
// Arithmetic (the reference's INT4 GEMV, tools/cmdlist/kernels.cpp:148-201,
// restated for bf16 activations): y[m][n] = sum_g s[n][g] * sum_{k in g}
// q[n][k] * x[m][k].  Here the inner sum runs on bf16 MFMA
// (v_mfma_f32_16x16x32_bf16): each packed nibble becomes the bf16 value
// 136 + q (bit pattern 0x4300 | (q + 8), two nibbles per AND-OR), the
// accumulator of every 128-wide group starts at -136 * sum_{k in g} x[m][k]
// (that sum comes from the same MFMA against a ones operand), so after the
// group's four MFMAs it holds sum q*x exactly as fp32 would, and the group
// scale is applied once per group in fp32.
//
// Tile: 16 tokens (MFMA M) x 16 weight rows (MFMA N).  Lane l owns weight
// row l%16 and k-quarter l/16 of every 128-wide group: one 16-byte load per
// lane per group and row-tile, coalesced 64-byte runs per row.  A block has
// WK x WR waves: WK waves split K (4 groups each, A kept in registers), WR
// waves take different row tiles; partial sums meet in LDS.
#include "moe_common.h"
#include "moe_internal.h"

namespace {

constexpr int KBW = 4;          // 128-wide groups per wave
constexpr int MAX_WAVES = 16;   // 1024 threads

__device__ __forceinline__ u32x4 ldg16(const void *p) {
  return __builtin_nontemporal_load((const u32x4 *)p);
}
__device__ __forceinline__ u32x4 ld16(const void *p) { return *(const u32x4 *)p; }

__device__ __forceinline__ u32x4 nib_slice(u32x4 b, int j) {
  return u32x4{nib_pair_bf16(b[0], j), nib_pair_bf16(b[1], j), nib_pair_bf16(b[2], j),
               nib_pair_bf16(b[3], j)};
}

__device__ __forceinline__ float silu_mul(float g, float u) {
  return g / (1.0f + expf(-g)) * u;
}

template <int SD, int MODE>
__global__ __launch_bounds__(1024) void k_expert_small(ExpertArgs a, int WK, int WR) {
  __shared__ float red[2][MAX_WAVES][256];
  const int tile_id = blockIdx.x;
  if (tile_id >= *a.n_tiles) return;
  const int2 tile = a.tiles[tile_id];
  const int e = tile.x, m0 = tile.y;
  const bool shared = e == a.E;
  // per-tile dimensions: MODE 0 rows = I (or Is), K = H; MODE 1 rows = H, K = I (or Is)
  const int N = MODE == 0 ? (shared ? a.Is : a.I) : a.H;
  const int K = MODE == 0 ? a.H : (shared ? a.Is : a.I);
  const int KB = K >> 7;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int kw = wave % WK, wr = wave / WK;
  const int n0 = (blockIdx.y * WR + wr) * 16;
  // whole block leaves together when it has no rows (uniform per block)
  if (blockIdx.y * WR * 16 >= N) return;

  int mcnt, pos0;
  if (shared) {
    mcnt = min(SMALL_MT, a.T - m0);
    pos0 = m0;
  } else {
    const int beg = a.offsets[e], cnt = a.offsets[e + 1] - beg;
    mcnt = min(SMALL_MT, cnt - m0);
    pos0 = beg + m0;
  }
  const int m = lane & 15, q = lane >> 4;
  const int kb0 = kw * KBW;
  const int nkb = max(0, min(KBW, KB - kb0));

  // ---- A operand (16 tokens x this wave's K range) into registers --------
  const uint16_t *arow = nullptr;
  if (m < mcnt) {
    if (MODE == 0) {
      int tok = shared ? m0 + m : a.perm[pos0 + m] / a.k;
      arow = a.a_routed + (size_t)tok * a.H;
    } else {
      arow = shared ? a.a_shared + (size_t)(m0 + m) * K : a.a_routed + (size_t)(pos0 + m) * K;
    }
  }
  u32x4 A[KBW][4];
#pragma unroll
  for (int i = 0; i < KBW; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      A[i][j] = u32x4{0u, 0u, 0u, 0u};
      if (arow && i < nkb) A[i][j] = ld16(arow + (size_t)(kb0 + i) * 128 + q * 32 + j * 8);
    }

  const bool active = n0 < N && nkb > 0;
  const int n = n0 + m;  // this lane's weight row (B operand column)
  f32x4 tot0 = {0.f, 0.f, 0.f, 0.f}, tot1 = {0.f, 0.f, 0.f, 0.f};
  if (active) {
    const uint8_t *w0 = shared ? a.ws0 : a.w0 + (size_t)e * N * (K / 2);
    const uint16_t *s0 = shared ? a.ss0 : a.s0 + (size_t)e * N * KB;
    const uint8_t *w1 = nullptr;
    const uint16_t *s1 = nullptr;
    if (MODE == 0) {
      w1 = shared ? a.ws1 : a.w1 + (size_t)e * N * (K / 2);
      s1 = shared ? a.ss1 : a.s1 + (size_t)e * N * KB;
    }
    // issue every weight load of this wave first
    u32x4 B0[KBW], B1[KBW];
    uint16_t S0[KBW], S1[KBW];
    const size_t rb = (size_t)n * (K / 2) + q * 16;
#pragma unroll
    for (int i = 0; i < KBW; ++i) {
      if (i < nkb) {
        B0[i] = ldg16(w0 + rb + (size_t)(kb0 + i) * 64);
        S0[i] = s0[(size_t)n * KB + kb0 + i];
        if (MODE == 0) {
          B1[i] = ldg16(w1 + rb + (size_t)(kb0 + i) * 64);
          S1[i] = s1[(size_t)n * KB + kb0 + i];
        }
      }
    }
    // group sums of A via a ones operand: lane gets sum for tokens 4q+r
    const u32x4 ones = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};
#pragma unroll
    for (int i = 0; i < KBW; ++i) {
      if (i < nkb) {
        f32x4 xs = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j) xs = mfma_bf16_16x16x32(A[i][j], ones, xs);
        const f32x4 c0 = xs * -136.0f;
        {
          const u32x4 b = B0[i] ^ 0x88888888u;
          f32x4 acc = c0;
#pragma unroll
          for (int j = 0; j < 4; ++j) acc = mfma_bf16_16x16x32(A[i][j], nib_slice(b, j), acc);
          const float s = scale_to_f32<SD>(S0[i]);
#pragma unroll
          for (int r = 0; r < 4; ++r) tot0[r] = __builtin_fmaf(s, acc[r], tot0[r]);
        }
        if (MODE == 0) {
          const u32x4 b = B1[i] ^ 0x88888888u;
          f32x4 acc = c0;
#pragma unroll
          for (int j = 0; j < 4; ++j) acc = mfma_bf16_16x16x32(A[i][j], nib_slice(b, j), acc);
          const float s = scale_to_f32<SD>(S1[i]);
#pragma unroll
          for (int r = 0; r < 4; ++r) tot1[r] = __builtin_fmaf(s, acc[r], tot1[r]);
        }
      }
    }
  }

  // ---- reduce the K split: D layout lane (q, m) holds rows 4q+r, col m ---
  const int nw = WK * WR;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    red[0][wave][(4 * q + r) * 16 + m] = tot0[r];
    if (MODE == 0) red[1][wave][(4 * q + r) * 16 + m] = tot1[r];
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < WR * 256; idx += nw * 64) {
    const int rwr = idx >> 8, cell = idx & 255;
    const int tm = cell >> 4, tn = cell & 15;
    const int row = (blockIdx.y * WR + rwr) * 16 + tn;
    if (tm >= mcnt || row >= N) continue;
    float g = 0.f, u = 0.f;
    for (int w = 0; w < WK; ++w) {
      g += red[0][rwr * WK + w][cell];
      if (MODE == 0) u += red[1][rwr * WK + w][cell];
    }
    if (MODE == 0) {
      const float v = silu_mul(g, u);
      if (shared)
        a.act_s[(size_t)(m0 + tm) * N + perm32_pos(row)] = f32_to_bf16(v);
      else
        a.act[(size_t)(pos0 + tm) * N + perm32_pos(row)] = f32_to_bf16(v);
    } else {
      const size_t orow = shared ? (size_t)a.T * a.k + m0 + tm : (size_t)(pos0 + tm);
      a.o[orow * a.H + row] = g;
    }
  }
}

}  // namespace

hipError_t launch_expert_small(int mode, int scale_dtype, const ExpertArgs &a, int max_tiles,
                               hipStream_t s) {
  if (max_tiles <= 0) return hipSuccess;
  const int Kr = mode == 0 ? a.H : a.I;
  const int Ks = mode == 0 ? a.H : a.Is;
  const int Nmax = mode == 0 ? (a.I > a.Is ? a.I : a.Is) : a.H;
  const int KBmax = (Kr > Ks ? Kr : Ks) / 128;
  int WK = (KBmax + KBW - 1) / KBW;
  if (WK < 1) WK = 1;
  if (WK > MAX_WAVES) return hipErrorInvalidValue;
  int WR = 4 / WK;
  if (WR < 1) WR = 1;
  const int threads = WK * WR * 64;
  dim3 grid(max_tiles, (Nmax + 16 * WR - 1) / (16 * WR));
  if (mode == 0) {
    if (scale_dtype == AINFER_SCALE_FP16)
      k_expert_small<AINFER_SCALE_FP16, 0><<<grid, threads, 0, s>>>(a, WK, WR);
    else
      k_expert_small<AINFER_SCALE_BF16, 0><<<grid, threads, 0, s>>>(a, WK, WR);
  } else {
    if (scale_dtype == AINFER_SCALE_FP16)
      k_expert_small<AINFER_SCALE_FP16, 1><<<grid, threads, 0, s>>>(a, WK, WR);
    else
      k_expert_small<AINFER_SCALE_BF16, 1><<<grid, threads, 0, s>>>(a, WK, WR);
  }
  return hipGetLastError();
}
