// moe_dispatch.h - the decode-size dispatch run by one block (T <= 64).
// Per-expert 64-bit token masks in LDS (order-free atomic OR), counts, an
// exclusive scan, the tile list, perm / inv / ptok, and the zeroing of the
// combine arrival counters.  Ranks come from popcounts of lower token bits,
// never from the order atomics land in.
#pragma once
#include "moe_common.h"
#include "moe_internal.h"

// 256 threads, T <= 64.
__device__ __forceinline__ void dispatch_small_block(const int32_t *__restrict__ idx, int T, int k, int E,
                                     int has_shared, const DispatchOut &ds) {
  __shared__ unsigned long long mask[1024];
  __shared__ int scan_c[256], scan_t[256];
  __shared__ int off_lds[1024];
  const int tid = threadIdx.x, mt = ds.mt;  // tokens per tile (T / mt <= 256)
  for (int e = tid; e < E; e += 256) mask[e] = 0ull;
  __syncthreads();
  for (int i = tid; i < T * k; i += 256)
    atomicOr(&mask[__builtin_nontemporal_load(idx + i)], 1ull << (i / k));
  __syncthreads();
  // per-thread contiguous expert range [e0, e0 + per)
  const int per = (E + 255) / 256;
  const int e0 = tid * per;
  int c_loc = 0, t_loc = 0;
  for (int e = e0; e < e0 + per && e < E; ++e) {
    const int c = __popcll(mask[e]);
    c_loc += c;
    t_loc += (c + mt - 1) / mt;
  }
  scan_c[tid] = c_loc;
  scan_t[tid] = t_loc;
  __syncthreads();
  for (int off = 1; off < 256; off <<= 1) {
    const int a = tid >= off ? scan_c[tid - off] : 0;
    const int b = tid >= off ? scan_t[tid - off] : 0;
    __syncthreads();
    scan_c[tid] += a;
    scan_t[tid] += b;
    __syncthreads();
  }
  int off_e = scan_c[tid] - c_loc, tile = scan_t[tid] - t_loc;
  for (int e = e0; e < e0 + per && e < E; ++e) {
    const int c = __popcll(mask[e]);
    ds.counts[e] = c;
    ds.offsets[e] = off_e;
    off_lds[e] = off_e;
    for (int m0 = 0; m0 < c; m0 += mt) ds.tiles[tile++] = make_int4(e, off_e + m0, min(mt, c - m0), 0);
    off_e += c;
  }
  const int routed_tiles = scan_t[255];
  if (tid == 0) ds.offsets[E] = scan_c[255];
  const int nsh = has_shared ? (T + mt - 1) / mt : 0;
  if (tid < nsh) ds.tiles[routed_tiles + tid] = make_int4(E, tid * mt, min(mt, T - tid * mt), 0);
  if (tid == 0) *ds.n_tiles = routed_tiles + nsh;
  __syncthreads();
  // placement: rank of token t among the tokens of expert e
  for (int i = tid; i < T * k; i += 256) {
    const int t = i / k;
    const int e = __builtin_nontemporal_load(idx + i);
    const unsigned long long below = t == 0 ? 0ull : ((~0ull) >> (64 - t));
    const int pos = off_lds[e] + __popcll(mask[e] & below);
    ds.perm[pos] = i;
    ds.inv[i] = pos;
    ds.ptok[pos] = t;
  }
}
