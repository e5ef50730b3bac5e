// moe_expert_item.h - one work item of the decode expert kernels: a tile of
// at most MT tokens routed to one expert x one slab of 16*RG*WR weight rows
// (moe_expert.hip describes the arithmetic and the tiling).  Shared by the
// stand-alone expert kernel (k_expert_lds) and the fused decode expert
// kernel (moe_decode.hip).
#pragma once
#include "moe_common.h"
#include "moe_internal.h"

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
// the same copy read device-coherently (sc1): data another workgroup wrote
// in this kernel
__device__ __forceinline__ void dma16_dev(const void *g, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off sc1"
               :
               : "v"(g), "s"(lds_addr)
               : "memory", "m0");
}

// Decode variant for tiles of at most MT tokens (MT = 4): the same work
// item and arithmetic as k_expert, but each wave copies its tile rows
// (MT tokens x its KBW k-groups, MT * KBW * 256 bytes) into a private LDS
// region with global->LDS DMA before the weight loads, and reads the A
// fragments from LDS per k-group.  A then holds no registers while the
// weight loads are in flight (more waves per SIMD) and costs MT * KBW / 4
// vector-memory instructions instead of 4 * KBW.  Rows past the tile's
// token count are copies of its last row; their results are never stored.
struct NoWait {
  __device__ void operator()() const {}
};

// COH: the outputs are read later in the same kernel by other workgroups
// (write them with sc1 stores).  COH_IN: the A rows were written earlier in
// the same kernel by other workgroups (read them with sc1).  Only wave 0
// returns from a COH item with work left (its stores still in flight); the
// LDS it needs is nw * MT * KBW * 256 bytes.
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
  float *red = (float *)(lds + nw * AW);  // K-split partial sums [2][nw][RG][256]
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
    const uint8_t *src;
    if (MODE == 0) {
      const int tok = shared ? pos0 + r : a.ptok[pos0 + r];
      src = (const uint8_t *)(a.a_routed + (size_t)tok * a.H);
    } else {
      src = (const uint8_t *)((shared ? a.a_shared : a.a_routed) + (size_t)(pos0 + r) * K);
    }
    asrc[d] = src + kb0 * 256 + c;
  }
  // ---- weight loads ------------------------------------------------------
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
#pragma unroll
  for (int g = 0; g < RG; ++g) {
    const int n = act ? min(n0 + g * 16 + m, N - 1) : m;
    const size_t rb = (size_t)n * rowb + q * 16;
#pragma unroll
    for (int i = 0; i < KBW; ++i) B0[g][i] = ldg_stream(w0 + rb + (size_t)(kb0 + i) * 64);
    load_scales<KBW>(s0 + (size_t)n * KB + kb0, S0[g]);
    if (MODE == 0) {
#pragma unroll
      for (int i = 0; i < KBW; ++i) B1[g][i] = ldg_stream(w1 + rb + (size_t)(kb0 + i) * 64);
      load_scales<KBW>(s1 + (size_t)n * KB + kb0, S1[g]);
    }
  }
  wait();
  // ---- A: this wave's tile rows -> LDS (row r at r * AROW), issued after the
  // weight loads; their sources were resolved before them ---------------------
  if (act) {
#pragma unroll
    for (int d = 0; d < AW / 1024; ++d) {
      if (COH_IN)
        dma16_dev(asrc[d], alds + d * 1024);
      else
        dma16(asrc[d], alds + d * 1024);
    }
  }
  // every load and DMA of this wave has landed
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // ---- MFMA ---------------------------------------------------------------
  f32x4 tot0[RG], tot1[RG];
#pragma unroll
  for (int g = 0; g < RG; ++g) tot0[g] = tot1[g] = f32x4{0.f, 0.f, 0.f, 0.f};
  if (act) {
    uint32_t magic;
    asm volatile("v_mov_b32 %0, 0x43004300" : "=v"(magic));
    const u32x4 ones = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};
    const uint8_t *arow = lds + wave * AW + (m % MT) * AROW + q * 64;
#pragma unroll
    for (int i = 0; i < KBW; ++i) {
      u32x4 A[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) A[j] = *(const u32x4 *)(arow + i * 256 + j * 16);
      f32x4 xs = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 4; ++j) xs = mfma_bf16_16x16x32(A[j], ones, xs);
      const f32x4 c0 = xs * -136.0f;
#pragma unroll
      for (int g = 0; g < RG; ++g) {
        {
          const u32x4 b = B0[g][i] ^ 0x88888888u;
          f32x4 acc = c0;
#pragma unroll
          for (int j = 0; j < 4; ++j) acc = mfma_bf16_16x16x32(A[j], nib_slice(b, j, magic), acc);
          tot0[g] += scale_to_f32<SD>(S0[g][i]) * acc;
        }
        if (MODE == 0) {
          const u32x4 b = B1[g][i] ^ 0x88888888u;
          f32x4 acc = c0;
#pragma unroll
          for (int j = 0; j < 4; ++j) acc = mfma_bf16_16x16x32(A[j], nib_slice(b, j, magic), acc);
          tot1[g] += scale_to_f32<SD>(S1[g][i]) * acc;
        }
      }
    }
  }
  // ---- K split meets in LDS: D layout lane (q, m) holds tokens 4q+r, row m.
  // COH: each wave's partials overwrite its own A region (its A reads have
  // completed: the MFMAs consumed them), and wave 0 alone finishes the item
  // while the other waves exit.
  // (when a wave's partials do not fit its A region they go past all A
  // regions: PART bytes per wave)
  constexpr int PART = (MODE == 0 ? 2 : 1) * RG * 1024;
  auto part = [&](int w, int half) -> float * {
    if (ALIAS)
      return (float *)(AW >= PART ? lds + w * AW : lds + nw * AW + w * PART) + half * RG * 256;
    return red + (half * nw + w) * RG * 256;
  };
#pragma unroll
  for (int g = 0; g < RG; ++g)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      part(wave, 0)[g * 256 + (4 * q + r) * 16 + m] = tot0[g][r];
      if (MODE == 0) part(wave, 1)[g * 256 + (4 * q + r) * 16 + m] = tot1[g][r];
    }
  __syncthreads();
  if (ALIAS && wave != 0) return;
  // tokens < mcnt <= MT only
  const int nthr = ALIAS ? 64 : nw * 64;
  for (int idx = ALIAS ? lane : (int)threadIdx.x; idx < a.WR * RG * 16 * MT; idx += nthr) {
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

