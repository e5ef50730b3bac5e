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
// One block = one work item: a tile of <= 16 tokens routed to one expert x
// 16*WR weight rows.  Each wave owns one 16-row group and KBW (1, 2 or 4)
// 128-wide k-groups; the WK waves of a row group meet in LDS.  Lane l owns
// weight row l%16 and k-quarter l/16 of every group: one 16-byte load per
// lane per group and matrix.
//
// Why this shape on MI355X: decode is bound by weight bytes in flight, so
// every wave issues all its weight loads at once and the waves per SIMD
// (register count) set the rate.  Larger batches use more k-groups per wave.
// Every branch is wave-uniform and no load is predicated, so each wave issues
// its loads back to back; token rows past the tile's count are read through
// a buffer descriptor at an out-of-range offset, which returns zeros
// without touching memory.
//
// MODE 0: gate and up together, epilogue silu(g)*u -> act (bf16, MFMA
//         order).
// MODE 1: down, epilogue o (bf16) per dispatch position; the combine kernel
//         sums a token's k + 1 rows in slot order.
#include <hip/hip_ext.h>

#include "moe_common.h"
#include "moe_internal.h"
#include "moe_expert_item.h"

namespace {

constexpr int MAX_WAVES = 16;  // 1024 threads

template <int SD, int KBW, int RG, int MODE>
__global__ __launch_bounds__(1024) void k_expert(ExpertArgs a) {
  // K-split partial sums: [2][waves][RG][256] floats (dynamic)
  extern __shared__ float red[];
  const int nw = a.WK * a.WR;
  const int n_rg = a.n_slabs;  // slabs of 16*RG*WR rows per tile
  const int tile_id = blockIdx.x / n_rg, slab = blockIdx.x % n_rg;
  if (tile_id >= *a.n_tiles) return;
  const int4 t = a.tiles[tile_id];
  const int e = t.x, pos0 = t.y, mcnt = t.z;
  const bool shared = e == a.E;
  const int N = MODE == 0 ? (shared ? a.Is : a.I) : a.H;
  const int K = MODE == 0 ? a.H : (shared ? a.Is : a.I);
  const int KB = K >> 7;
  if (slab * a.WR * RG * 16 >= N) return;

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int kw = wave % a.WK, wr = wave / a.WK;
  const int m = lane & 15, q = lane >> 4;
  const int n0 = (slab * a.WR + wr) * RG * 16;  // first of this wave's RG row groups
  // wave-uniform: this wave has rows and k-groups in this item
  const bool act = n0 < N && kw * KBW < KB;
  const int kb0 = act ? kw * KBW : 0;

  // ---- A row of this lane's token (a buffer offset; lanes past the tile's
  // token count get an out-of-range offset and read zeros) ----------------
  const int mm = min(m, mcnt - 1);
  uint32_t aoff;
  const uint16_t *abase;
  if (MODE == 0) {
    const int tok = shared ? pos0 + mm : a.ptok[pos0 + mm];
    abase = a.a_routed;
    aoff = (uint32_t)tok * (uint32_t)a.H * 2u;  // < T * H * 2 <= 2^29
  } else {
    // the tile's first row moves the (uniform) base in 64-bit arithmetic, so
    // the 32-bit buffer offset only spans the tile: (T*k) * I * 2 bytes can
    // pass 2^31 at large T, the tile's 16 rows never do
    abase = (shared ? a.a_shared : a.a_routed) + (size_t)pos0 * K;
    aoff = (uint32_t)mm * (uint32_t)K * 2u;
  }
  if (m >= mcnt) aoff = BUF_OOB;
  const __amdgpu_buffer_rsrc_t arsrc = make_rsrc(abase, 0x7FFFFFFFu);
  // ---- weight loads: RG row groups x KBW k-groups (rows past N are clamped:
  // their results are never stored) ------------------------------------------
  const size_t rowb = (size_t)K / 2;
  const uint8_t *w0 = shared ? a.ws0 : a.w0 + (size_t)e * N * rowb;
  const uint16_t *s0 = shared ? a.ss0 : a.s0 + (size_t)e * N * KB;
  const uint8_t *w1 = nullptr;
  const uint16_t *s1 = nullptr;
  if (MODE == 0) {
    w1 = shared ? a.ws1 : a.w1 + (size_t)e * N * rowb;
    s1 = shared ? a.ss1 : a.s1 + (size_t)e * N * KB;
  }
  u32x4 B0[RG][KBW], B1[RG][KBW];
  uint16_t S0[RG][KBW], S1[RG][KBW];
  // Wide pattern (KBW = 4): a row's KBW * 64 bytes are LPR = 4 KBW lanes of
  // one global->LDS DMA instruction (16 / KBW rows per instruction instead of
  // 16 rows x 64 B), which streams from HBM faster; the lanes then read their
  // MFMA fragments (row m, quarter q of group i) back from LDS.  16-byte
  // chunk c of row r sits at chunk c ^ (r % LPR): the 16 rows one fragment
  // read touches at one logical chunk land on distinct bank groups.
  constexpr int LPR = 4 * KBW, RPI = 64 / LPR, MATS = MODE == 0 ? 2 : 1;
  constexpr int WROWB = LPR * 16;  // staged bytes per row
  uint8_t *bst = (uint8_t *)red + (size_t)2 * nw * RG * 256 * sizeof(float) +
                 (size_t)wave * MATS * RG * 16 * WROWB;
  if constexpr (KBW >= 4) {
    const uint32_t bl = (uint32_t)(uintptr_t)bst;
#pragma unroll
    for (int mat = 0; mat < MATS; ++mat)
#pragma unroll
      for (int g = 0; g < RG; ++g)
#pragma unroll
        for (int j = 0; j < KBW; ++j) {
          const int r = j * RPI + lane / LPR, pc = lane % LPR;
          const int c = pc ^ (r % LPR);
          const int n = act ? min(n0 + g * 16 + r, N - 1) : r;
          const uint8_t *src = (mat ? w1 : w0) + (size_t)n * rowb + (size_t)kb0 * 64 + c * 16;
          dma16(src, __builtin_amdgcn_readfirstlane(bl + (uint32_t)(((mat * RG + g) * 16 + j * RPI) * WROWB)));
        }
  }
#pragma unroll
  for (int g = 0; g < RG; ++g) {
    const int n = act ? min(n0 + g * 16 + m, N - 1) : m;
    const size_t rb = (size_t)n * rowb + q * 16;
    if constexpr (KBW < 4) {
#pragma unroll
      for (int i = 0; i < KBW; ++i) B0[g][i] = ldg_stream(w0 + rb + (size_t)(kb0 + i) * 64);
      if (MODE == 0)
#pragma unroll
        for (int i = 0; i < KBW; ++i) B1[g][i] = ldg_stream(w1 + rb + (size_t)(kb0 + i) * 64);
    }
    load_scales<KBW>(s0 + (size_t)n * KB + kb0, S0[g]);
    if (MODE == 0) load_scales<KBW>(s1 + (size_t)n * KB + kb0, S1[g]);
  }
  u32x4 A[KBW][4];
#pragma unroll
  for (int i = 0; i < KBW; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      A[i][j] = buf_load16(arsrc, aoff + (uint32_t)(((kb0 + i) * 128 + q * 32 + j * 8) * 2));

  if constexpr (KBW >= 4) {
    // this wave's DMA (and every load above) has landed
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
    for (int g = 0; g < RG; ++g)
#pragma unroll
      for (int i = 0; i < KBW; ++i) {
        const int pc = (i * 4 + q) ^ (m % LPR);
        B0[g][i] = *(const u32x4 *)(bst + (size_t)(g * 16 + m) * WROWB + pc * 16);
        if (MODE == 0) B1[g][i] = *(const u32x4 *)(bst + (size_t)((RG + g) * 16 + m) * WROWB + pc * 16);
      }
  }
  // ---- MFMA ---------------------------------------------------------------
  f32x4 tot0[RG], tot1[RG];
#pragma unroll
  for (int g = 0; g < RG; ++g) tot0[g] = tot1[g] = f32x4{0.f, 0.f, 0.f, 0.f};
  if (act) {
    uint32_t magic;
    asm volatile("v_mov_b32 %0, 0x43004300" : "=v"(magic));
    const u32x4 ones = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};
#pragma unroll
    for (int i = 0; i < KBW; ++i) {
      f32x4 xs = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 4; ++j) xs = mfma_bf16_16x16x32(A[i][j], ones, xs);
      const f32x4 c0 = xs * -136.0f;
#pragma unroll
      for (int g = 0; g < RG; ++g) {
        {
          const u32x4 b = B0[g][i] ^ 0x88888888u;
          f32x4 acc = c0;
#pragma unroll
          for (int j = 0; j < 4; ++j) acc = mfma_bf16_16x16x32(A[i][j], nib_slice(b, j, magic), acc);
          tot0[g] += scale_to_f32<SD>(S0[g][i]) * acc;
        }
        if (MODE == 0) {
          const u32x4 b = B1[g][i] ^ 0x88888888u;
          f32x4 acc = c0;
#pragma unroll
          for (int j = 0; j < 4; ++j) acc = mfma_bf16_16x16x32(A[i][j], nib_slice(b, j, magic), acc);
          tot1[g] += scale_to_f32<SD>(S1[g][i]) * acc;
        }
      }
    }
  }
  // ---- K split meets in LDS: D layout lane (q, m) holds tokens 4q+r, row m
  float *red0 = red, *red1 = red + nw * RG * 256;
#pragma unroll
  for (int g = 0; g < RG; ++g)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      red0[(wave * RG + g) * 256 + (4 * q + r) * 16 + m] = tot0[g][r];
      if (MODE == 0) red1[(wave * RG + g) * 256 + (4 * q + r) * 16 + m] = tot1[g][r];
    }
  __syncthreads();
  const int nthr = nw * 64;
  for (int idx = threadIdx.x; idx < a.WR * RG * 256; idx += nthr) {
    const int rgrp = idx >> 8, cell = idx & 255;  // rgrp = wr * RG + g
    const int rwr = rgrp / RG, g = rgrp % RG;
    const int tm = cell >> 4, tn = cell & 15;
    const int row = (slab * a.WR + rwr) * RG * 16 + g * 16 + tn;
    if (tm >= mcnt || row >= N) continue;
    float gs = 0.f, u = 0.f;
    for (int w = 0; w < a.WK; ++w) {
      const int src = ((rwr * a.WK + w) * RG + g) * 256 + cell;
      gs += red0[src];
      if (MODE == 0) u += red1[src];
    }
    if (MODE == 0) {
      uint16_t *dst = shared ? a.act_s : a.act;
      dst[(size_t)(pos0 + tm) * N + perm32_pos(row)] = f32_to_bf16(silu_mul(gs, u));
    } else {
      const size_t orow = shared ? (size_t)a.T * a.k + pos0 + tm : (size_t)(pos0 + tm);
      a.o[orow * a.H + row] = f32_to_bf16(gs);
    }
  }
}



template <int SD, int KBW, int RG, int MT, int MODE>
__global__ __launch_bounds__(1024) void k_expert_lds(ExpertArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int tile_id = blockIdx.x / a.n_slabs, slab = blockIdx.x % a.n_slabs;
  int n_tiles;
  const int4 t = sload_tile(a.tiles, a.n_tiles, tile_id, n_tiles);
  if (tile_id >= n_tiles) return;
  expert_lds_item<SD, KBW, RG, MT, MODE, false, false, true>(a, t, slab, lds);
}

}  // namespace

#ifdef AINFER_DECODE_TRACE
extern "C" int ainfer_debug_land_expert(void *host) {
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(g_dland), sizeof(g_dland)) == hipSuccess ? 0 : -1;
}
#endif

// KBW k-groups per wave (the preferred count, raised until one row group
// fits in 16 waves, lowered until it divides both K group counts), WK =
// waves along K, WR = row groups per block.
#ifndef EXPERT_WAVES
#define EXPERT_WAVES 4  // waves per expert item (K-split x row groups)
#endif
bool expert_geometry(int mode, int H, int I, int Is, int pref_kbw, int *KBW, int *WK,
                     int *WR) {
  const int KBr = (mode == 0 ? H : I) / 128;
  const int KBs = (mode == 0 ? H : (Is > 0 ? Is : I)) / 128;
  const int KBmax = KBr > KBs ? KBr : KBs;
  int kbw = pref_kbw < 1 ? 1 : (pref_kbw > 4 ? 4 : pref_kbw);
  while ((KBmax + kbw - 1) / kbw > MAX_WAVES && kbw < 4) kbw *= 2;
  while (kbw > 1 && (KBr % kbw || KBs % kbw)) kbw /= 2;
  if ((KBmax + kbw - 1) / kbw > MAX_WAVES || KBr % kbw || KBs % kbw) return false;
  const int wk = KBmax / kbw;
  int wr = EXPERT_WAVES / wk;
  if (wr < 1) wr = 1;
  *KBW = kbw;
  *WK = wk;
  *WR = wr;
  return true;
}


hipEvent_t g_kev_start = nullptr, g_kev_stop = nullptr;

template <int SD, int MODE, int RG>
void launch_kbw(int kbw, int mt, unsigned grid, int threads, size_t lds, const ExpertArgs &a,
                hipStream_t s) {
  if (mt == DEC_MT) {
    auto go = [&](auto kern) {
      if (g_kev_start) {  // profiling: the kernel's own start and end
        hipExtLaunchKernelGGL(kern, dim3(grid), dim3(threads), (uint32_t)lds, s, g_kev_start,
                              g_kev_stop, 0u, a);
        g_kev_start = g_kev_stop = nullptr;
      } else {
        kern<<<grid, threads, lds, s>>>(a);
      }
    };
    if (kbw == 1)
      go(k_expert_lds<SD, 1, RG, DEC_MT, MODE>);
    else if (kbw == 2)
      go(k_expert_lds<SD, 2, RG, DEC_MT, MODE>);
    else
      go(k_expert_lds<SD, 4, RG, DEC_MT, MODE>);
    return;
  }
  if (kbw == 1)
    k_expert<SD, 1, RG, MODE><<<grid, threads, lds, s>>>(a);
  else if (kbw == 2)
    k_expert<SD, 2, RG, MODE><<<grid, threads, lds, s>>>(a);
  else
    k_expert<SD, 4, RG, MODE><<<grid, threads, lds, s>>>(a);
}

template <int SD, int MODE>
void launch_rg(int rg, int kbw, int mt, unsigned grid, int threads, size_t lds,
               const ExpertArgs &a, hipStream_t s) {
  if (rg == 1)
    launch_kbw<SD, MODE, 1>(kbw, mt, grid, threads, lds, a, s);
  else if (rg == 2)
    launch_kbw<SD, MODE, 2>(kbw, mt, grid, threads, lds, a, s);
  else
    launch_kbw<SD, MODE, 4>(kbw, mt, grid, threads, lds, a, s);
}

void set_expert_launch_events(hipEvent_t start, hipEvent_t stop) {
  g_kev_start = start;
  g_kev_stop = stop;
}

hipError_t launch_expert_stream(int mode, int scale_dtype, ExpertArgs a, int max_tiles,
                                int pref_kbw, int rg, int mt, hipStream_t s) {
  if (max_tiles <= 0) return hipSuccess;
  if (rg != 1 && rg != 2 && rg != 4) return hipErrorInvalidValue;
  if (mt != DEC_MT && mt != SMALL_MT) return hipErrorInvalidValue;
  int kbw;
  if (!expert_geometry(mode, a.H, a.I, a.Is, pref_kbw, &kbw, &a.WK, &a.WR))
    return hipErrorInvalidValue;
  const int Nmax = mode == 0 ? (a.I > a.Is ? a.I : a.Is) : a.H;
  a.n_slabs = (Nmax + 16 * rg * a.WR - 1) / (16 * rg * a.WR);
  const int threads = a.WK * a.WR * 64;
  size_t lds = sizeof(float) * 2 * (size_t)a.WK * a.WR * rg * 256;
  if (kbw >= 4)  // the wide B staging of k_expert: per wave (mats x RG x 16 rows x KBW * 64 B)
    lds += (size_t)a.WK * a.WR * (mode == 0 ? 2 : 1) * rg * 16 * kbw * 64;
  if (mt == DEC_MT) {
    // A staging; the K-split partials reuse it when they fit (expert_lds_item, ALIAS)
    lds = (size_t)a.WK * a.WR * item_lds_per_wave(DEC_MT, kbw, rg, mode);
  }
  if (lds > 160 * 1024) return hipErrorInvalidValue;
  const long grid = (long)max_tiles * a.n_slabs;
  if (grid > 0x7FFFFFFF) return hipErrorInvalidValue;
  if (mode == 0) {
    if (scale_dtype == AINFER_SCALE_FP16)
      launch_rg<AINFER_SCALE_FP16, 0>(rg, kbw, mt, (unsigned)grid, threads, lds, a, s);
    else
      launch_rg<AINFER_SCALE_BF16, 0>(rg, kbw, mt, (unsigned)grid, threads, lds, a, s);
  } else {
    if (scale_dtype == AINFER_SCALE_FP16)
      launch_rg<AINFER_SCALE_FP16, 1>(rg, kbw, mt, (unsigned)grid, threads, lds, a, s);
    else
      launch_rg<AINFER_SCALE_BF16, 1>(rg, kbw, mt, (unsigned)grid, threads, lds, a, s);
  }
  return hipGetLastError();
}
