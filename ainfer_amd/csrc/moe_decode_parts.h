// moe_decode_parts.h - device pieces shared by the decode kernels
// (moe_decode.hip) and the persistent decode-stack kernel (moe_stack.hip):
// bounded waits, a scalar-cache tile load, and the one-workgroup dispatch of
// a few tokens.
#pragma once
#include "moe_common.h"
#include "moe_internal.h"

namespace {

__device__ __forceinline__ bool spin_until_geq(const int32_t *p, int target, int spin) {
  for (int it = 0; it < spin; ++it) {
    if (__hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= target) return true;
    __builtin_amdgcn_s_sleep(8);
  }
  return false;
}

// Workgroup-wide: thread 0 polls.  What the awaited workgroups published is
// then read with sc1 loads (moe_common.h).
__device__ __forceinline__ void block_wait_geq(const int32_t *p, int target, int32_t *err,
                                               int spin) {
  if (threadIdx.x == 0 && !spin_until_geq(p, target, spin)) atomicOr(err, 1);
  __syncthreads();
}

// A uniform 16-byte load through the scalar cache (the compiler cannot
// prove the tile list read-only inside this kernel and would use a vector
// load, whose wait also waits for every weight load in flight).
__device__ __forceinline__ int4 sload_int4(const int4 *p) {
  typedef int i32x4 __attribute__((ext_vector_type(4)));
  i32x4 v;
  asm volatile("s_load_dwordx4 %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(p) : "memory");
  return make_int4(v[0], v[1], v[2], v[3]);
}

// Dispatch of T <= 32 tokens by one workgroup (idx in LDS): 32-bit token masks
// per expert (order-free atomic OR), counts, a workgroup exclusive scan over
// experts, tiles of at most DEC_MT tokens, perm / inv / ptok.
template <int W>
__device__ __forceinline__ void dispatch_decode(const int32_t *__restrict__ idx, int T, int k,
                                                int E, int has_shared, const DispatchOut &ds) {
  __shared__ uint32_t msk[1024];
  __shared__ int offl[1024];
  __shared__ int wsum[W];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  if (T == 1 && k <= 64) {
    // One token: the k picks are distinct experts, each a one-token tile.
    // Pick j's position is its rank among the picks by expert index (the
    // general path's expert-order scan); wave 0 alone, no barrier.
    if (wv != 0) return;
    const int e = lane < k ? idx[lane] : 0x7FFFFFFF;
    int r = 0;
    for (int j = 0; j < k; ++j) r += __builtin_amdgcn_readlane(e, j) < e ? 1 : 0;
    if (lane < k) {
      ds.tiles[r] = make_int4(e, r, 1, 0);
      ds.perm[r] = lane;
      ds.inv[lane] = r;
      ds.ptok[r] = 0;
    }
    if (lane == 0) {
      if (has_shared) ds.tiles[k] = make_int4(E, 0, 1, 0);
      *ds.n_tiles = k + (has_shared ? 1 : 0);
      if (ds.offsets) ds.offsets[E] = k;
    }
    if (ds.counts) {
      for (int ee = lane; ee < E; ee += 64) {
        int below = 0, hit = 0;
        for (int j = 0; j < k; ++j) {
          const int ej = __builtin_amdgcn_readlane(e, j);
          below += ej < ee ? 1 : 0;
          hit |= ej == ee ? 1 : 0;
        }
        ds.counts[ee] = hit;
        ds.offsets[ee] = below;
      }
    }
    return;
  }
  constexpr int NT = W * 64;
  for (int e = tid; e < E; e += NT) msk[e] = 0u;
  __syncthreads();
  for (int i = tid; i < T * k; i += NT) atomicOr(&msk[idx[i]], 1u << (i / k));
  __syncthreads();
  const int per = (E + NT - 1) / NT;
  const int e0 = tid * per, e1 = min(e0 + per, E);
  int c_loc = 0, t_loc = 0;
  for (int e = e0; e < e1; ++e) {
    const int c = __popc(msk[e]);
    c_loc += c;
    t_loc += (c + DEC_MT - 1) / DEC_MT;
  }
  // one scan of (tiles << 16 | tokens): both stay below 2^16 (T * k entries)
  const int packed = wave_scan_incl((t_loc << 16) | c_loc);
  if (lane == 63) wsum[wv] = packed;
  __syncthreads();
  int base = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < W; ++w) {
    const int v = wsum[w];
    base += w < wv ? v : 0;
    tot += v;
  }
  const int cb = base & 0xFFFF, tb0 = base >> 16, ctot = tot & 0xFFFF, ttot = tot >> 16;
  const int ci = packed & 0xFFFF, ti = packed >> 16;
  int o = cb + ci - c_loc, tb = tb0 + ti - t_loc;
  for (int e = e0; e < e1; ++e) {
    const int c = __popc(msk[e]);
    if (ds.counts) {  // null: only the tiles and positions are wanted
      ds.counts[e] = c;
      ds.offsets[e] = o;
    }
    offl[e] = o;
    for (int m0 = 0; m0 < c; m0 += DEC_MT) ds.tiles[tb++] = make_int4(e, o + m0, min(DEC_MT, c - m0), 0);
    o += c;
  }
  const int nsh = has_shared ? (T + DEC_MT - 1) / DEC_MT : 0;
  if (tid < nsh) ds.tiles[ttot + tid] = make_int4(E, tid * DEC_MT, min(DEC_MT, T - tid * DEC_MT), 0);
  if (tid == 0) {
    if (ds.offsets) ds.offsets[E] = ctot;
    *ds.n_tiles = ttot + nsh;
  }
  __syncthreads();
  for (int i = tid; i < T * k; i += NT) {
    const int t = i / k, e = idx[i];
    const int pos = offl[e] + __popc(msk[e] & ((1u << t) - 1u));
    ds.perm[pos] = i;
    ds.inv[i] = pos;
    ds.ptok[pos] = t;
  }
}

}  // namespace
