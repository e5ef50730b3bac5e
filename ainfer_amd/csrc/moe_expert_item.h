// moe_expert_item.h - one work item of the decode expert kernels: a tile of
// at most MT tokens routed to one expert x one slab of 16*RG*WR weight rows
// (moe_expert.hip describes the INT4 arithmetic).  Shared by the
// stand-alone expert kernel (k_expert_lds) and the fused decode expert
// kernel (moe_decode.hip).
#pragma once
#include "moe_common.h"
#include "moe_internal.h"

#ifdef AINFER_DECODE_TRACE
// debug builds only: per workgroup, when its item started, its wave 0's
// weight loads landed, and its partials were written
static __device__ unsigned long long g_dland[2][1 << 14][3];  // [MODE][workgroup]
#define ITRACE(I) \
  if (threadIdx.x == 0 && blockIdx.x < (1 << 14)) g_dland[MODE][blockIdx.x][I] = __builtin_amdgcn_s_memrealtime()
#else
#define ITRACE(I)
#endif

// A tile entry and the tile count in one scalar round trip: both loads are
// in flight before the wait (a count read first, then the entry, costs two
// trips while every workgroup of the launch reads the same lines).  `tile`
// is below the launch's tile bound, so the entry is inside the tile list
// whether or not the dispatch filled it; the caller checks it against n.
__device__ __forceinline__ int4 sload_tile(const int4 *tiles, const int32_t *n_tiles, int tile,
                                           int &n) {
  typedef int i32x4 __attribute__((ext_vector_type(4)));
  i32x4 v;
  int c;
  asm volatile("s_load_dword %1, %3, 0x0\n\ts_load_dwordx4 %0, %2, 0x0\n\ts_waitcnt lgkmcnt(0)"
               : "=&s"(v), "=&s"(c)
               : "s"(tiles + tile), "s"(n_tiles)
               : "memory");
  n = c;
  return make_int4(v[0], v[1], v[2], v[3]);
}

__device__ __forceinline__ u32x4 ldg_stream(const void *p) {
  return __builtin_nontemporal_load((const u32x4 *)p);
}

// Four bf16 pairs (136 + q) for MFMA k-slice j of a 16-byte chunk already
// xor'ed with 0x88888888.  `magic` is 0x43004300 held in a register so the
// AND-OR is a single instruction.
__device__ __forceinline__ u32x4 nib_slice(u32x4 b, int j, uint32_t magic) {
  const uint32_t mask = 0x000F000Fu;
  return u32x4{((b[0] >> (4 * j)) & mask) | magic, ((b[1] >> (4 * j)) & mask) | magic,
               ((b[2] >> (4 * j)) & mask) | magic, ((b[3] >> (4 * j)) & mask) | magic};
}

// The KBW scales of one row and k-range in one load (KB is a multiple of
// KBW, so the address is KBW * 2-byte aligned).
template <int KBW>
__device__ __forceinline__ void load_scales(const uint16_t *p, uint16_t (&S)[KBW]) {
  if constexpr (KBW == 4) {
    const uint2 v = *(const uint2 *)p;
    S[0] = (uint16_t)v.x; S[1] = (uint16_t)(v.x >> 16);
    S[2] = (uint16_t)v.y; S[3] = (uint16_t)(v.y >> 16);
  } else if constexpr (KBW == 2) {
    const uint32_t v = *(const uint32_t *)p;
    S[0] = (uint16_t)v; S[1] = (uint16_t)(v >> 16);
  } else {
    S[0] = *p;
  }
}

__device__ __forceinline__ float silu_mul(float g, float u) {
  return g / (1.0f + expf(-g)) * u;
}

__device__ __forceinline__ void dma16(const void *g, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(g), "s"(lds_addr)
               : "memory", "m0");
}
// one dword per lane (256 bytes per instruction) into LDS
__device__ __forceinline__ void dma4(const void *g, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off"
               :
               : "v"(g), "s"(lds_addr)
               : "memory", "m0");
}
// the same copy read device-coherently (sc1): data another workgroup wrote
// in this kernel
__device__ __forceinline__ void dma16_dev(const void *g, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off sc1"
               :
               : "v"(g), "s"(lds_addr)
               : "memory", "m0");
}

// Decode item for tiles of at most MT = 4 tokens: one expert x one slab of
// 16 * RG * WR weight rows, WK waves along K.  Each wave:
//  - loads its weights 4 rows x 256 bytes per instruction (16 / KBW rows x
//    KBW * 64 B): lane (r4, b) holds 32 nibbles of row r4 of row quad
//    b / CPR at chunk b % CPR, exactly the B operand of block b of
//    v_mfma_f32_4x4x4bf16_1k.  Wide row segments stream from HBM about 15%
//    faster than the 16 rows x 64 B a 16x16x32 operand would take;
//  - copies its scales (one dword DMA per 256 B) and the tile's token rows
//    (MT * KBW * 256 B, only the instructions holding a row below the token
//    count) into LDS with global->LDS DMA, so neither holds registers while
//    the weights are in flight;
//  - runs 8 MFMAs per weight register (4 tokens x 4 k per block, no token
//    padding), scales each block's sums by its row's group scale, and sums
//    the CPR chunks of a row across lanes by halving (permlane swaps and
//    ds_swizzle).
// The K split meets in LDS; the token-row order in HBM (the MFMA order of
// moe_common.h) is shared with the prefill kernels.
struct NoWait {
  __device__ void operator()() const {}
};

// COH: the outputs are read later in the same kernel by other workgroups
// (write them with sc1 stores).  COH_IN: the A rows were written earlier in
// the same kernel by other workgroups (read them with sc1).  Only wave 0
// returns from a COH item with work left (its stores still in flight); the
// LDS it needs is nw * item_lds_per_wave(MT, KBW, RG, MODE) bytes.
// wait(): called by every thread after the weight loads are issued and
// before the A rows are read (the weights never depend on earlier work).
template <int SD, int KBW, int RG, int MT, int MODE, bool COH = false, bool COH_IN = COH,
          bool ALIAS = COH, typename Wait = NoWait>
__device__ __forceinline__ void expert_lds_item(const ExpertArgs &a, int4 t, int slab,
                                                uint8_t *lds, Wait wait = Wait()) {
  constexpr int AROW = KBW * 256;  // bytes of one token row in this wave's k-range
  constexpr int AW = MT * AROW;    // LDS bytes per wave
  static_assert(AW % 1024 == 0, "one DMA instruction moves 1 KB");
  const int nw = a.WK * a.WR;
  // LDS: [nw][AW] A rows, [nw][SCB] scales, then the partial sums
  constexpr int SCB = item_scale_lds(KBW, RG, MODE);
  float *red = (float *)(lds + nw * (AW + SCB));  // K-split partial sums [2][nw][RG][256]
  ITRACE(0);
  const int e = t.x, pos0 = t.y, mcnt = t.z;
  const bool shared = e == a.E;
  const int N = MODE == 0 ? (shared ? a.Is : a.I) : a.H;
  const int K = MODE == 0 ? a.H : (shared ? a.Is : a.I);
  const int KB = K >> 7;
  if (slab * a.WR * RG * 16 >= N) return;

  const int tx = tid_opaque();
  const int wave = __builtin_amdgcn_readfirstlane(tx >> 6);
  const int lane = tx & 63;
  const int kw = wave % a.WK, wr = wave / a.WK;
  const int m = lane & 15, q = lane >> 4;
  const int n0 = (slab * a.WR + wr) * RG * 16;
  const bool act = n0 < N && kw * KBW < KB;
  const int kb0 = act ? kw * KBW : 0;
  const uint32_t alds = (uint32_t)(uintptr_t)lds + (uint32_t)(wave * AW);

  // ---- sources of the A copy (the token ids are loaded first: waiting for
  // them later must not wait for the weight loads) --------------------------
  const uint8_t *asrc[AW / 1024];
#pragma unroll
  for (int d = 0; d < AW / 1024; ++d) {
    const int off = d * 1024 + lane * 16, r = min(off / AROW, mcnt - 1), c = off % AROW;
    asrc[d] = nullptr;
    if (d * 1024 >= mcnt * AROW) continue;  // not copied
    const uint8_t *src;
    if (MODE == 0) {
      const int tok = shared ? pos0 + r : a.ptok[pos0 + r];
      src = (const uint8_t *)(a.a_routed + (size_t)tok * a.H);
    } else {
      src = (const uint8_t *)((shared ? a.a_shared : a.a_routed) + (size_t)(pos0 + r) * K);
    }
    asrc[d] = src + kb0 * 256 + c;
  }
  // ---- weight loads: one instruction covers 16 / KBW rows x KBW * 64 bytes
  // (4 rows x 256 B at KBW = 4).  Lane (r4, b): row quad b / CPR, row r4 of
  // it, 16-byte chunk c = b % CPR of the wave's k-range: the B operand of the
  // 4x4x4 MFMA's block b (row r4, 32 k of chunk c) --------------------------
  const size_t rowb = (size_t)K / 2;
  const uint8_t *w0 = shared ? a.ws0 : a.w0 + (size_t)e * N * rowb;
  const uint16_t *s0 = shared ? a.ss0 : a.s0 + (size_t)e * N * KB;
  const uint8_t *w1 = nullptr;
  const uint16_t *s1 = nullptr;
  if (MODE == 0) {
    w1 = shared ? a.ws1 : a.w1 + (size_t)e * N * rowb;
    s1 = shared ? a.ss1 : a.s1 + (size_t)e * N * KB;
  }
  constexpr int CPR = 4 * KBW;   // 32-k chunks of a row in the wave's k-range
  constexpr int RPI = 16 / KBW;  // rows per load instruction
  constexpr int U = RG * KBW;    // load instructions per matrix
  const int r4 = lane & 3, c = (lane >> 2) % CPR, rq = (lane >> 2) / CPR;
  u32x4 B0[U], B1[U];
  uint16_t S0[U], S1[U];
  // scales (KBW >= 2): dword d of [mat][row of the wave's RG * 16][KBW]
  // scales, one DMA per 64 dwords, issued after the weight loads
  const uint32_t slds = (uint32_t)(uintptr_t)lds + (uint32_t)(nw * AW + wave * SCB);
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int n = act ? min(n0 + u * RPI + 4 * rq + r4, N - 1) : r4;
    const size_t rb = (size_t)n * rowb + (size_t)kb0 * 64 + c * 16;
    const size_t sb = (size_t)n * KB + kb0 + (c >> 2);
    B0[u] = ldg_stream(w0 + rb);
    if constexpr (KBW == 1) S0[u] = s0[sb];
    if (MODE == 0) {
      B1[u] = ldg_stream(w1 + rb);
      if constexpr (KBW == 1) S1[u] = s1[sb];
    }
  }
  if constexpr (KBW >= 2) {
    constexpr int DPR = KBW / 2, DPM = RG * 16 * DPR;  // dwords per row, per matrix
#pragma unroll
    for (int i = 0; i < (MODE == 0 ? 2 : 1) * DPM; i += 64) {
      const int d = min(i + lane, (MODE == 0 ? 2 : 1) * DPM - 1);
      const int mat = d / DPM, rw = (d % DPM) / DPR, dw = d % DPR;
      const int n = act ? min(n0 + rw, N - 1) : 0;
      const uint16_t *sp = (mat ? s1 : s0) + (size_t)n * KB + kb0 + 2 * dw;
      dma4(sp, __builtin_amdgcn_readfirstlane(slds + i * 4));
    }
  }
  wait();
  // ---- A: this wave's tile rows -> LDS (row r at r * AROW), issued after the
  // weight loads; their sources were resolved before them ---------------------
  // (only the instructions that hold a row below mcnt: the MFMA reads row
  // min(t, mcnt - 1) for token t)
  if (act) {
#pragma unroll
    for (int d = 0; d < AW / 1024; ++d) {
      if (d * 1024 >= mcnt * AROW) break;
      if (COH_IN)
        dma16_dev(asrc[d], alds + d * 1024);
      else
        dma16(asrc[d], alds + d * 1024);
    }
  }
  // every load and DMA of this wave has landed
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  ITRACE(1);
  if constexpr (KBW >= 2) {
    const uint16_t *sl = (const uint16_t *)(lds + nw * AW + wave * SCB);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int rw = u * RPI + 4 * rq + r4, j = rw * KBW + (c >> 2);
      S0[u] = sl[j];
      if (MODE == 0) S1[u] = sl[RG * 16 * KBW + j];
    }
  }

  // ---- MFMA: v_mfma_f32_4x4x4bf16_1k, A = 4 tokens x 4 k (lane (t, b) reads
  // 8 bytes of token row t of the MFMA-ordered tile), B = 4 rows x 4 k per
  // block, D lane (r4, b) register t: row r4, token t, the k of chunk c.
  // Nibbles become bf16 136 + q (moe_common.h); the 136 * sum(x) term is
  // taken off through an MFMA with a ones operand.  One row and one k-group
  // per lane, so each result is scaled by one scale ------------------------
  constexpr int MATS = MODE == 0 ? 2 : 1;
  constexpr int V = MATS * U * 4;  // partial sums (mat, u, token) of this lane
  // MODE 0 halves at once over the top lane bit: gate and up of one (u,
  // token) are the pair the first halving step adds, so the lane keeps VH
  constexpr int VH = MODE == 0 ? V / 2 : V;
  float v[VH];
#pragma unroll
  for (int i = 0; i < VH; ++i) v[i] = 0.0f;
  if (act) {
    uint32_t magic;
    asm volatile("v_mov_b32 %0, 0x43004300" : "=v"(magic));
    const uint8_t *xa = lds + wave * AW + min(r4, mcnt - 1) * AROW + c * 64;
    s16x4 A[8];  // (j, half): x positions 8 j + 4 half + [0, 4) of chunk c
#pragma unroll
    for (int jh = 0; jh < 8; ++jh) A[jh] = *(const s16x4 *)(xa + jh * 8);
    const s16x4 ones = {0x3F80, 0x3F80, 0x3F80, 0x3F80};
    f32x4 xs = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int jh = 0; jh < 8; ++jh) xs = mfma_bf16_4x4x4(A[jh], ones, xs);
    const f32x4 c0 = xs * -136.0f;
    const uint32_t mask = 0x000F000Fu;
    auto dot = [&](const u32x4 bw0, uint16_t sraw) {
      const u32x4 bw = bw0 ^ 0x88888888u;
      f32x4 acc = c0;
#pragma unroll
      for (int jh = 0; jh < 8; ++jh) {
        const int j = jh >> 1, h = jh & 1;
        const uint32_t d0 = ((bw[2 * h] >> (4 * j)) & mask) | magic;
        const uint32_t d1 = ((bw[2 * h + 1] >> (4 * j)) & mask) | magic;
        acc = mfma_bf16_4x4x4(A[jh], __builtin_bit_cast(s16x4, u32x2{d0, d1}), acc);
      }
      return acc * scale_to_f32<SD>(sraw);
    };
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const f32x4 g = dot(B0[u], S0[u]);
      if constexpr (MODE == 0) {
        const f32x4 up = dot(B1[u], S1[u]);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          float p[2] = {g[t], up[t]};
          HalveSum<2, 2 * CPR>::step(p, lane);
          v[u * 4 + t] = p[0];
        }
      } else {
#pragma unroll
        for (int t = 0; t < 4; ++t) v[u * 4 + t] = g[t];
      }
    }
  }
  // ---- sum over the CPR chunks of a row (lane bits 2 .. 1 + log2 CPR),
  // halving the values at each step: afterwards lane (r4, b) holds the
  // F = V / CPR sums of original indices c * F + i --------------------------
  constexpr int F = V / CPR;
  static_assert(F >= 1, "at least one sum per lane");
  if constexpr (MODE == 0)
    HalveSum<VH, CPR>::run(v, lane);
  else
    HalveSum<VH, 2 * CPR>::run(v, lane);
  // ---- K split meets in LDS: partials [g][token][row of 16] as the 16 x 16
  // MFMA's D layout placed them.  COH: each wave's partials overwrite its own
  // A region (its A reads have completed: the MFMAs consumed them), and wave
  // 0 alone finishes the item while the other waves exit.
  // (when a wave's partials do not fit its A region they go past all A
  // regions: PART bytes per wave)
  constexpr int PART = (MODE == 0 ? 2 : 1) * RG * 1024;
  auto part = [&](int w, int half) -> float * {
    if (ALIAS)
      return (float *)(AW >= PART ? lds + w * AW : lds + nw * (AW + SCB) + w * PART) + half * RG * 256;
    return red + (half * nw + w) * RG * 256;
  };
#pragma unroll
  for (int i = 0; i < F; ++i) {
    const int o = c * F + i, t = o & 3, mu = o >> 2, u = mu % U, mat = mu / U;
    const int rw = u * RPI + 4 * rq + r4;  // row within the wave's RG * 16
    part(wave, mat)[(rw >> 4) * 256 + t * 16 + (rw & 15)] = v[i];
  }
  ITRACE(2);
  __syncthreads();
  if (ALIAS && wave != 0) return;
  // tokens < mcnt <= MT only
  const int nthr = ALIAS ? 64 : nw * 64;
  for (int idx = ALIAS ? lane : tx; idx < a.WR * RG * 16 * MT; idx += nthr) {
    const int rgrp = idx / (16 * MT), cell = idx % (16 * MT);  // rgrp = wr * RG + g
    const int rwr = rgrp / RG, g = rgrp % RG;
    const int tm = cell >> 4, tn = cell & 15;
    const int row = (slab * a.WR + rwr) * RG * 16 + g * 16 + tn;
    if (tm >= mcnt || row >= N) continue;
    float gs = 0.f, u = 0.f;
    for (int w = 0; w < a.WK; ++w) {
      gs += part(rwr * a.WK + w, 0)[g * 256 + cell];
      if (MODE == 0) u += part(rwr * a.WK + w, 1)[g * 256 + cell];
    }
    if (MODE == 0) {
      uint16_t *dst = shared ? a.act_s : a.act;
      const size_t i = (size_t)(pos0 + tm) * N + perm32_pos(row);
      const uint16_t v = f32_to_bf16(silu_mul(gs, u));
      if (COH)
        st_dev_u16(make_rsrc(dst, 0x7FFFFFFFu), (uint32_t)(i * 2), v);
      else
        dst[i] = v;
    } else {
      const size_t orow = shared ? (size_t)a.T * a.k + pos0 + tm : (size_t)(pos0 + tm);
      const uint16_t v = f32_to_bf16(gs);
      if (COH)
        st_dev_u16(make_rsrc(a.o, 0x7FFFFFFFu), (uint32_t)((orow * a.H + row) * 2), v);
      else
        a.o[orow * a.H + row] = v;
    }
  }
}

