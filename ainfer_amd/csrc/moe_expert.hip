// moe_expert.hip - grouped INT4 expert kernels for small token tiles (decode).
//
// Arithmetic (the reference's INT4 GEMV, tools/cmdlist/kernels.cpp:148-201,
// restated for bf16 activations): y[m][n] = sum_g s[n][g] * sum_{k in g}
// q[n][k] * x[m][k].  The inner sum runs on bf16 MFMA
// (v_mfma_f32_16x16x32_bf16): each packed nibble becomes the bf16 value
// 136 + q (bit pattern 0x4300 | (q + 8), two nibbles per AND-OR), the
// accumulator of every 128-wide group starts at -136 * sum_{k in g} x[m][k]
// (that sum comes from the same MFMA against a ones operand), so after the
// group's four MFMAs it holds sum q*x, and the group scale is applied once
// per group in fp32.
//
// Work item = (token tile of <= 16 rows of one expert, slab of 16*WR weight
// rows).  A block of WK x WR waves owns a contiguous range of items: WK waves
// split K (4 groups each, A operand kept in registers for the whole tile),
// WR waves take different 16-row groups.  Lane l owns weight row l%16 and
// k-quarter l/16 of every group: one 16-byte load per lane per group.  The
// weight loads of item i+1 are in flight while item i computes.
//
// MODE 0: gate and up together, epilogue silu(g)*u -> act (bf16, MFMA
//         order).
// MODE 1: down, epilogue o (fp32); then per (token, slab) an arrival
//         counter: the block that brings the last of the token's k + 1
//         contributions sums them in slot order (+ shared, + residual) and
//         writes y.  The sum order never depends on which block arrives last.
#include "moe_common.h"
#include "moe_internal.h"

namespace {

constexpr int KBW = 4;        // 128-wide groups per wave
constexpr int MAX_WAVES = 8;  // 512 threads

__device__ __forceinline__ u32x4 ldg_stream(const void *p) {
  return __builtin_nontemporal_load((const u32x4 *)p);
}

__device__ __forceinline__ u32x4 nib_slice(u32x4 b, int j) {
  return u32x4{nib_pair_bf16(b[0], j), nib_pair_bf16(b[1], j), nib_pair_bf16(b[2], j),
               nib_pair_bf16(b[3], j)};
}

__device__ __forceinline__ float silu_mul(float g, float u) {
  return g / (1.0f + expf(-g)) * u;
}

struct TileState {
  int id = -1;
  int e, pos0, mcnt, m0;
  bool shared;
  int N, K, KB, nkb, kb0;
};

template <int MODE>
__device__ __forceinline__ void tile_load(const ExpertArgs &a, int tile_id, int kw,
                                          TileState &ts) {
  const int4 t = a.tiles[tile_id];
  ts.id = tile_id;
  ts.e = t.x;
  ts.pos0 = t.y;
  ts.mcnt = t.z;
  ts.m0 = t.w;
  ts.shared = t.x == a.E;
  ts.N = MODE == 0 ? (ts.shared ? a.Is : a.I) : a.H;
  ts.K = MODE == 0 ? a.H : (ts.shared ? a.Is : a.I);
  ts.KB = ts.K >> 7;
  ts.kb0 = kw * KBW;
  ts.nkb = max(0, min(KBW, ts.KB - ts.kb0));
}

// A operand of this wave's K range for the tile's tokens, and the -136 *
// group-sum accumulator starts (D layout: tokens 4q+r).
template <int MODE>
__device__ __forceinline__ void a_load(const ExpertArgs &a, const TileState &ts, int lane,
                                       u32x4 (&A)[KBW][4], f32x4 (&C0)[KBW]) {
  const int m = lane & 15, q = lane >> 4;
  const uint16_t *arow = nullptr;
  if (m < ts.mcnt) {
    if (MODE == 0) {
      const int tok = ts.shared ? ts.pos0 + m : a.ptok[ts.pos0 + m];
      arow = a.a_routed + (size_t)tok * a.H;
    } else {
      arow = ts.shared ? a.a_shared + (size_t)(ts.pos0 + m) * ts.K
                       : a.a_routed + (size_t)(ts.pos0 + m) * ts.K;
    }
  }
#pragma unroll
  for (int i = 0; i < KBW; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      A[i][j] = u32x4{0u, 0u, 0u, 0u};
      if (arow && i < ts.nkb)
        A[i][j] = *(const u32x4 *)(arow + (size_t)(ts.kb0 + i) * 128 + q * 32 + j * 8);
    }
  const u32x4 ones = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};
#pragma unroll
  for (int i = 0; i < KBW; ++i) {
    f32x4 xs = {0.f, 0.f, 0.f, 0.f};
    if (i < ts.nkb) {
#pragma unroll
      for (int j = 0; j < 4; ++j) xs = mfma_bf16_16x16x32(A[i][j], ones, xs);
    }
    C0[i] = xs * -136.0f;
  }
}

template <int MODE>
__device__ __forceinline__ void b_issue(const ExpertArgs &a, const TileState &ts, int slab,
                                        int wr, int lane, u32x4 (&B0)[KBW], u32x4 (&B1)[KBW],
                                        uint16_t (&S0)[KBW], uint16_t (&S1)[KBW]) {
  const int m = lane & 15, q = lane >> 4;
  const int n0 = (slab * a.WR + wr) * 16;
  if (n0 >= ts.N || ts.nkb == 0) return;
  const int n = n0 + m;
  const size_t rowb = (size_t)ts.K / 2;
  const uint8_t *w0 = ts.shared ? a.ws0 : a.w0 + (size_t)ts.e * ts.N * rowb;
  const uint16_t *s0 = ts.shared ? a.ss0 : a.s0 + (size_t)ts.e * ts.N * ts.KB;
  const size_t rb = (size_t)n * rowb + q * 16;
#pragma unroll
  for (int i = 0; i < KBW; ++i)
    if (i < ts.nkb) {
      B0[i] = ldg_stream(w0 + rb + (size_t)(ts.kb0 + i) * 64);
      S0[i] = s0[(size_t)n * ts.KB + ts.kb0 + i];
    }
  if (MODE == 0) {
    const uint8_t *w1 = ts.shared ? a.ws1 : a.w1 + (size_t)ts.e * ts.N * rowb;
    const uint16_t *s1 = ts.shared ? a.ss1 : a.s1 + (size_t)ts.e * ts.N * ts.KB;
#pragma unroll
    for (int i = 0; i < KBW; ++i)
      if (i < ts.nkb) {
        B1[i] = ldg_stream(w1 + rb + (size_t)(ts.kb0 + i) * 64);
        S1[i] = s1[(size_t)n * ts.KB + ts.kb0 + i];
      }
  }
}

template <int SD, int MODE>
__device__ __forceinline__ void mma_item(const TileState &ts, const u32x4 (&A)[KBW][4],
                                         const f32x4 (&C0)[KBW], const u32x4 (&B0)[KBW],
                                         const u32x4 (&B1)[KBW], const uint16_t (&S0)[KBW],
                                         const uint16_t (&S1)[KBW], f32x4 &tot0, f32x4 &tot1) {
  tot0 = f32x4{0.f, 0.f, 0.f, 0.f};
  tot1 = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < KBW; ++i) {
    if (i < ts.nkb) {
      {
        const u32x4 b = B0[i] ^ 0x88888888u;
        f32x4 acc = C0[i];
#pragma unroll
        for (int j = 0; j < 4; ++j) acc = mfma_bf16_16x16x32(A[i][j], nib_slice(b, j), acc);
        const float s = scale_to_f32<SD>(S0[i]);
#pragma unroll
        for (int r = 0; r < 4; ++r) tot0[r] = __builtin_fmaf(s, acc[r], tot0[r]);
      }
      if (MODE == 0) {
        const u32x4 b = B1[i] ^ 0x88888888u;
        f32x4 acc = C0[i];
#pragma unroll
        for (int j = 0; j < 4; ++j) acc = mfma_bf16_16x16x32(A[i][j], nib_slice(b, j), acc);
        const float s = scale_to_f32<SD>(S1[i]);
#pragma unroll
        for (int r = 0; r < 4; ++r) tot1[r] = __builtin_fmaf(s, acc[r], tot1[r]);
      }
    }
  }
}

template <int MODE>
__device__ __forceinline__ void epilogue(const ExpertArgs &a, const TileState &ts, int slab,
                                         int wave, int lane, const f32x4 &tot0,
                                         const f32x4 &tot1, float (*red)[MAX_WAVES][256],
                                         int *s_done, int *s_ndone) {
  const int m = lane & 15, q = lane >> 4;
  const int WK = a.WK, WR = a.WR, nthr = WK * WR * 64;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    red[0][wave][(4 * q + r) * 16 + m] = tot0[r];
    if (MODE == 0) red[1][wave][(4 * q + r) * 16 + m] = tot1[r];
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < WR * 256; idx += nthr) {
    const int rwr = idx >> 8, cell = idx & 255;
    const int tm = cell >> 4, tn = cell & 15;
    const int row = (slab * WR + rwr) * 16 + tn;
    if (tm >= ts.mcnt || row >= ts.N) continue;
    float g = 0.f, u = 0.f;
    for (int w = 0; w < WK; ++w) {
      g += red[0][rwr * WK + w][cell];
      if (MODE == 0) u += red[1][rwr * WK + w][cell];
    }
    if (MODE == 0) {
      const float v = silu_mul(g, u);
      uint16_t *dst = ts.shared ? a.act_s : a.act;
      dst[(size_t)(ts.pos0 + tm) * ts.N + perm32_pos(row)] = f32_to_bf16(v);
    } else {
      const size_t orow = ts.shared ? (size_t)a.T * a.k + ts.pos0 + tm : (size_t)(ts.pos0 + tm);
      a.o[orow * a.H + row] = g;
    }
  }
  if (MODE == 1) {
    // ---- arrival counting and the slot-order combine -------------------
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) *s_ndone = 0;
    __syncthreads();
    const int need = a.k + (a.has_shared ? 1 : 0);
    if ((int)threadIdx.x < ts.mcnt) {
      const int tok = ts.shared ? ts.pos0 + threadIdx.x : a.ptok[ts.pos0 + threadIdx.x];
      const int old = atomicAdd(&a.cnt[tok * a.n_slabs + slab], 1);
      if (old == need - 1) {
        const int slot = atomicAdd(s_ndone, 1);
        s_done[slot] = tok;
      }
    }
    __syncthreads();
    const int nd = *s_ndone;
    if (nd > 0) {
      __threadfence();
      const int rows = WR * 16, r0 = slab * rows;
      for (int idx = threadIdx.x; idx < nd * rows; idx += nthr) {
        const int tok = s_done[idx / rows], row = r0 + idx % rows;
        if (row >= a.H) continue;
        float acc = 0.0f;
        for (int j = 0; j < a.k; ++j) {
          const int p = a.inv[tok * a.k + j];
          acc = __builtin_fmaf(a.topk_w[tok * a.k + j], a.o[(size_t)p * a.H + row], acc);
        }
        if (a.has_shared)
          acc = __builtin_fmaf(a.sg[tok], a.o[((size_t)a.T * a.k + tok) * a.H + row], acc);
        if (a.resid) acc += bf16_to_f32(a.resid[(size_t)tok * a.H + row]);
        a.y[(size_t)tok * a.H + row] = f32_to_bf16(acc);
        if (idx % rows == 0) a.cnt[tok * a.n_slabs + slab] = 0;
      }
    }
  }
  __syncthreads();
}

template <int SD, int MODE>
__global__ __launch_bounds__(512) void k_expert_stream(ExpertArgs a) {
  __shared__ float red[2][MAX_WAVES][256];
  __shared__ int s_done[16];
  __shared__ int s_ndone;
  const int n_items = *a.n_tiles * a.n_slabs;
  const int G = gridDim.x, b = blockIdx.x;
  const int i0 = (int)((long)b * n_items / G), i1 = (int)((long)(b + 1) * n_items / G);
  if (i0 >= i1) return;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int kw = wave % a.WK, wr = wave / a.WK;

  TileState cur, nxt;
  u32x4 A[KBW][4];
  f32x4 C0[KBW];
  u32x4 PB0[KBW], PB1[KBW], QB0[KBW], QB1[KBW];
  uint16_t PS0[KBW], PS1[KBW], QS0[KBW], QS1[KBW];
  f32x4 tot0, tot1;

  tile_load<MODE>(a, i0 / a.n_slabs, kw, cur);
  b_issue<MODE>(a, cur, i0 % a.n_slabs, wr, lane, PB0, PB1, PS0, PS1);
  a_load<MODE>(a, cur, lane, A, C0);

  for (int i = i0; i < i1; i += 2) {
    // ---- item i (buffers P); item i+1 prefetched into Q ---------------
    const bool has1 = i + 1 < i1;
    if (has1) {
      const int t1 = (i + 1) / a.n_slabs;
      nxt = cur;
      if (t1 != cur.id) tile_load<MODE>(a, t1, kw, nxt);
      b_issue<MODE>(a, nxt, (i + 1) % a.n_slabs, wr, lane, QB0, QB1, QS0, QS1);
    }
    mma_item<SD, MODE>(cur, A, C0, PB0, PB1, PS0, PS1, tot0, tot1);
    epilogue<MODE>(a, cur, i % a.n_slabs, wave, lane, tot0, tot1, red, s_done, &s_ndone);
    if (!has1) break;
    if (nxt.id != cur.id) {
      cur = nxt;
      a_load<MODE>(a, cur, lane, A, C0);
    }
    // ---- item i+1 (buffers Q); item i+2 prefetched into P -------------
    const bool has2 = i + 2 < i1;
    if (has2) {
      const int t2 = (i + 2) / a.n_slabs;
      nxt = cur;
      if (t2 != cur.id) tile_load<MODE>(a, t2, kw, nxt);
      b_issue<MODE>(a, nxt, (i + 2) % a.n_slabs, wr, lane, PB0, PB1, PS0, PS1);
    }
    mma_item<SD, MODE>(cur, A, C0, QB0, QB1, QS0, QS1, tot0, tot1);
    epilogue<MODE>(a, cur, (i + 1) % a.n_slabs, wave, lane, tot0, tot1, red, s_done, &s_ndone);
    if (has2 && nxt.id != cur.id) {
      cur = nxt;
      a_load<MODE>(a, cur, lane, A, C0);
    }
  }
}

int g_num_cus = 0;

}  // namespace

void expert_geometry(int mode, const ExpertArgs &a, int *WK, int *WR) {
  const int Kr = mode == 0 ? a.H : a.I;
  const int Ks = mode == 0 ? a.H : (a.Is > 0 ? a.Is : a.I);
  const int KBmax = (Kr > Ks ? Kr : Ks) / 128;
  int wk = (KBmax + KBW - 1) / KBW;
  if (wk < 1) wk = 1;
  int wr = 4 / wk;
  if (wr < 1) wr = 1;
  *WK = wk;
  *WR = wr;
}

hipError_t launch_expert_stream(int mode, int scale_dtype, ExpertArgs a, int max_tiles,
                                hipStream_t s) {
  if (max_tiles <= 0) return hipSuccess;
  expert_geometry(mode, a, &a.WK, &a.WR);
  if (a.WK * a.WR > MAX_WAVES) return hipErrorInvalidValue;
  const int Nmax = mode == 0 ? (a.I > a.Is ? a.I : a.Is) : a.H;
  a.n_slabs = (Nmax + 16 * a.WR - 1) / (16 * a.WR);
  if (g_num_cus == 0) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&g_num_cus, hipDeviceAttributeMultiprocessorCount, dev) !=
            hipSuccess)
      g_num_cus = 256;
  }
  const int threads = a.WK * a.WR * 64;
  const long max_items = (long)max_tiles * a.n_slabs;
  const long per_cu = threads <= 256 ? 2 : 1;
  long grid = g_num_cus * per_cu;
  if (grid > max_items) grid = max_items;
  if (mode == 0) {
    if (scale_dtype == AINFER_SCALE_FP16)
      k_expert_stream<AINFER_SCALE_FP16, 0><<<(unsigned)grid, threads, 0, s>>>(a);
    else
      k_expert_stream<AINFER_SCALE_BF16, 0><<<(unsigned)grid, threads, 0, s>>>(a);
  } else {
    if (scale_dtype == AINFER_SCALE_FP16)
      k_expert_stream<AINFER_SCALE_FP16, 1><<<(unsigned)grid, threads, 0, s>>>(a);
    else
      k_expert_stream<AINFER_SCALE_BF16, 1><<<(unsigned)grid, threads, 0, s>>>(a);
  }
  return hipGetLastError();
}
