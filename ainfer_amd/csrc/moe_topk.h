// moe_topk.h - exact top-k of one token's E logits inside one wave (wave64).
//
// Order: value descending, equal values lower expert index first (the tie
// rule of tools/sample/sampler.h:97-98).  Lane l holds the ordered keys of
// experts l, l + 64, ... (ordered_key: unsigned order = float order).
#pragma once
#include "moe_common.h"

// inverse of ordered_key (-0 comes back as +0)
__device__ __forceinline__ float key_to_float(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

// k rounds of (largest key, then lowest expert among equal keys).  Lane
// j < k returns the j-th pick in seli and its key in selk; the return value
// is the k-th largest key.  Every lane keeps its best untaken slot; a round is one wave max,
// then the winner from a ballot (a second reduction over expert ids only
// when several lanes hold the maximum), and only the winning lane rescans.
template <int NV>
__device__ __forceinline__ uint32_t wave_topk(const uint32_t (&key)[NV], int E, int k, int lane,
                                              int &seli, uint32_t &selk) {
  uint32_t taken = 0;
#pragma unroll
  for (int i = 0; i < NV; ++i)
    if (lane + 64 * i >= E) taken |= 1u << i;
  uint32_t bk = 0;
  int bs = -1;
  auto rescan = [&]() {
    bk = 0;
    bs = -1;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const bool better = !((taken >> i) & 1u) && (bs < 0 || key[i] > bk);
      bk = better ? key[i] : bk;
      bs = better ? i : bs;
    }
  };
  rescan();
  uint32_t kth = 0;
  seli = 0;
  selk = 0;
  for (int j = 0; j < k; ++j) {
    const uint32_t wk = wave_max_u32(bs >= 0 ? bk : 0u);
    const bool hold = bs >= 0 && bk == wk;
    const uint64_t tie = __ballot(hold);
    uint32_t we;
    if (__popcll(tie) == 1) {
      const int wl = __builtin_ctzll(tie);
      we = (uint32_t)(wl + 64 * __builtin_amdgcn_readlane(bs, wl));
    } else {
      we = wave_min_u32(hold ? (uint32_t)(lane + 64 * bs) : 0xFFFFFFFFu);
    }
    if (lane == (int)(we & 63)) {
      taken |= 1u << (we >> 6);
      rescan();
    }
    if (lane == j) {
      seli = (int)we;
      selk = wk;
    }
    kth = wk;
  }
  return kth;
}

template <int CTRL>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t v) {
  const int lo = __builtin_amdgcn_update_dpp((int)(uint32_t)v, (int)(uint32_t)v, CTRL, 0xF, 0xF, false);
  const int hi = __builtin_amdgcn_update_dpp((int)(uint32_t)(v >> 32), (int)(uint32_t)(v >> 32), CTRL,
                                             0xF, 0xF, false);
  return ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo;
}
__device__ __forceinline__ uint64_t readlane_u64(uint64_t v, int l) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, l);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), l);
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

// Fast exact top-k for k <= 16.  Composite c = key << 32 | ~expert is
// unique per expert and orders exactly as the rule above (0 = absent).
//  1. tau = the k-th largest of the 16 quad maxima (each quad of lanes
//     covers 4 * NV experts).  The k quads whose maxima are >= tau hold k
//     distinct experts >= tau, so every expert of the top-k is >= tau.
//  2. Experts >= tau are compacted into `cand` (LDS, 64 entries per wave)
//     at offsets from a wave prefix sum of the per-lane counts; for random
//     logits there are about k + 5 of them.
//  3. Each candidate's rank is the number of candidates above it; rank
//     r < k is pick r.
// More than 64 candidates (many equal logits), an absent tau or k > 16 take
// the round-by-round path above.  Lane j < k returns pick j in seli and its
// key in selk.  cand and sel are wave-private LDS arrays (68 and 16 entries).
template <int NV>
__device__ __forceinline__ void wave_topk_fast(const uint32_t (&key)[NV], int E, int k, int lane,
                                               int &seli, uint32_t &selk, uint64_t *cand,
                                               uint64_t *sel) {
  if (k > 16) {
    wave_topk<NV>(key, E, k, lane, seli, selk);
    return;
  }
  uint64_t c[NV];
  uint64_t lm = 0;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int e = lane + 64 * i;
    c[i] = e < E ? (((uint64_t)key[i] << 32) | (uint32_t)~(uint32_t)e) : 0ull;
    lm = max_u64(lm, c[i]);
  }
  lm = max_u64(lm, dpp_u64<0xB1>(lm));  // quad_perm [1,0,3,2]
  lm = max_u64(lm, dpp_u64<0x4E>(lm));  // quad_perm [2,3,0,1]
  int r = 0;
#pragma unroll
  for (int q = 0; q < 16; ++q) r += readlane_u64(lm, 4 * q) > lm ? 1 : 0;
  const uint64_t tb = __ballot(r == k - 1);
  const uint64_t tau = tb ? readlane_u64(lm, __builtin_ctzll(tb)) : 0ull;
  int nc = 0;
  if (tau != 0ull) {
    // each lane's candidates at its offset from a wave prefix sum of the
    // per-lane counts (one scan instead of NV ballot rounds; the rank below
    // does not depend on the list's order)
    bool p[NV];
    int cnt = 0;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      p[i] = c[i] >= tau;
      cnt += p[i] ? 1 : 0;
    }
    const int incl = wave_scan_incl(cnt);
    nc = __builtin_amdgcn_readlane(incl, 63);
    int pos = incl - cnt;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      if (p[i] && pos < 64) cand[pos] = c[i];
      pos += p[i] ? 1 : 0;
    }
  }
  if (tau == 0ull || nc > 64) {
    wave_topk<NV>(key, E, k, lane, seli, selk);
    return;
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  const uint64_t mine = lane < nc ? cand[lane] : 0ull;
  int rk = 0;
  if (nc <= 16) {
    // the usual case (about k + 5 candidates): every broadcast read in
    // flight at once; entries past nc are ignored
    uint64_t v[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) v[j] = cand[j];
#pragma unroll
    for (int j = 0; j < 16; ++j) rk += (j < nc && v[j] > mine) ? 1 : 0;
  } else {
    // four broadcast reads in flight per step
    for (int j0 = 0; j0 < nc; j0 += 4) {
      uint64_t v[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] = cand[j0 + q];
#pragma unroll
      for (int q = 0; q < 4; ++q) rk += (j0 + q < nc && v[q] > mine) ? 1 : 0;
    }
  }
  if (lane < nc && rk < k) sel[rk] = mine;
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  const uint64_t pick = lane < k ? sel[lane] : 0ull;
  seli = lane < k ? (int)~(uint32_t)pick : 0;
  selk = (uint32_t)(pick >> 32);
}
