// moe_route.hip - router, top-k, dispatch, combine, RMSNorm and synthetic
// fill kernels for gfx950 (wave64).
//
// Router semantics (no counterpart in the reference, which is a dense model;
// tie rule from tools/sample/sampler.h:90-98): fp32 logits in the
// lane-strided chunk order, top-k by value with lower index first on ties,
// renormalised softmax weights over the selected k, sigmoid shared gate.
// Dispatch: expert-contiguous permutation, token ascending within an expert,
// built from per-64-token-chunk LDS bitmasks so ranks never depend on the
// order atomics land in.
#include <string.h>

#include "moe_common.h"
#include "moe_internal.h"

// ---------------------------------------------------------------------------
// synthetic fill (same definition as the CPU oracle's mo_fill)
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint64_t rnd64(uint64_t seed, uint64_t i) {
  uint64_t z = seed + (i + 1u) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
__device__ __forceinline__ float std_normal8(uint64_t r) {
  int s = 0;
#pragma unroll
  for (int b = 0; b < 8; ++b) s += (int)((r >> (8 * b)) & 0xFFu);
  return (float)(s - 1020) * 0x1.39897ep-8f;
}
// IEEE binary16 round-to-nearest-even, written out on integers.
__device__ __forceinline__ uint16_t f32_to_fp16_rne(float f) {
  uint32_t x = __float_as_uint(f);
  uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7FFFFFFFu;
  if (ax >= 0x7F800000u) return (uint16_t)(sign | (ax > 0x7F800000u ? 0x7E00u : 0x7C00u));
  if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);
  if (ax < 0x38800000u) {
    uint32_t e = ax >> 23;
    if (e < 102) return (uint16_t)sign;
    uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
    uint32_t shift = 126u - e;
    uint32_t r = m >> shift, rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (r & 1u))) r++;
    return (uint16_t)(sign | r);
  }
  uint32_t r = ax - 0x38000000u;
  uint32_t out = r >> 13, rem = r & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (out & 1u))) out++;
  return (uint16_t)(sign | out);
}

__global__ void k_fill_bytes(uint64_t seed, size_t n, uint8_t *out) {
  size_t nw = (n + 7) / 8;
  for (size_t w = blockIdx.x * (size_t)blockDim.x + threadIdx.x; w < nw;
       w += (size_t)gridDim.x * blockDim.x) {
    uint64_t r = rnd64(seed, w);
    if (w * 8 + 8 <= n && (((uintptr_t)out) & 7) == 0) {
      *(uint64_t *)(out + w * 8) = r;
    } else {
      for (int b = 0; b < 8 && w * 8 + b < n; ++b) out[w * 8 + b] = (uint8_t)(r >> (8 * b));
    }
  }
}
__global__ void k_fill_half(int kind, uint64_t seed, float std_, size_t n, uint16_t *out) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x) {
    float v = std_normal8(rnd64(seed, i)) * std_;
    uint16_t o;
    if (kind == AINFER_FILL_BF16_NORMAL) o = f32_to_bf16(v);
    else if (kind == AINFER_FILL_FP16_ABSNORMAL) o = f32_to_fp16_rne(fabsf(v));
    else o = f32_to_bf16(fabsf(v));
    out[i] = o;
  }
}

hipError_t launch_fill(int kind, uint64_t seed, float std_, size_t n, void *out,
                       hipStream_t s) {
  if (n == 0) return hipSuccess;
  const int threads = 256;
  size_t work = kind == AINFER_FILL_BYTES ? (n + 7) / 8 : n;
  size_t blocks = (work + threads - 1) / threads;
  if (blocks > 65536) blocks = 65536;
  if (kind == AINFER_FILL_BYTES)
    k_fill_bytes<<<(unsigned)blocks, threads, 0, s>>>(seed, n, (uint8_t *)out);
  else
    k_fill_half<<<(unsigned)blocks, threads, 0, s>>>(kind, seed, std_, n, (uint16_t *)out);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// RMSNorm: one 256-thread block per row; fp64 sum of squares in the fixed
// order lane-strided + pairwise tree (the shape of RMSNormW,
// tools/cmdlist/kernels.cpp:94-113), fp32 normalise, bf16 out.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_rmsnorm(const uint16_t *__restrict__ x,
                                                 const uint16_t *__restrict__ w, int mode,
                                                 float eps, uint16_t *__restrict__ y, int H) {
  __shared__ double ps[256];
  const int t = blockIdx.x, lid = threadIdx.x;
  const uint16_t *xr = x + (size_t)t * H;
  double ss = 0.0;
  for (int j = lid; j < H; j += 256) {
    double v = (double)bf16_to_f32(xr[j]);
    ss += v * v;
  }
  ps[lid] = ss;
  __syncthreads();
  for (int st = 128; st > 0; st >>= 1) {
    if (lid < st) ps[lid] += ps[lid + st];
    __syncthreads();
  }
  double tot = ps[0];
  float inv = 1.0f / sqrtf((float)(tot / H) + eps);
  for (int j = lid; j < H; j += 256) {
    float wt = 1.0f;
    if (w) {
      float wv = bf16_to_f32(w[j]);
      wt = mode == AINFER_NORM_ONE_PLUS ? 1.0f + wv : wv;
    }
    float v = bf16_to_f32(xr[j]) * inv;
    y[(size_t)t * H + j] = f32_to_bf16(v * wt);
  }
}

hipError_t launch_rmsnorm(const void *x, const void *w, int mode, float eps, void *y,
                          int T, int H, hipStream_t s) {
  if (T == 0) return hipSuccess;
  k_rmsnorm<<<T, 256, 0, s>>>((const uint16_t *)x, (const uint16_t *)w, mode, eps,
                              (uint16_t *)y, H);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Router logits.  One wave per weight row (E expert rows, then the shared
// gate row), TT tokens per pass.  Lane l covers 8-element chunks
// l, l+64, ... with sequential fma, then an xor butterfly: the
// lane-strided chunk order the CPU oracle restates.
// ---------------------------------------------------------------------------
constexpr int ROUTER_TT = 8;

__global__ __launch_bounds__(256) void k_router_logits(const uint16_t *__restrict__ x,
                                                       const uint16_t *__restrict__ rw,
                                                       const float *__restrict__ bias,
                                                       const uint16_t *__restrict__ gw,
                                                       float *__restrict__ logits,
                                                       float *__restrict__ sg_logit,
                                                       int32_t *__restrict__ ticket, int T,
                                                       int H, int E) {
  const int lane = threadIdx.x & 63;
  if (ticket && blockIdx.x == 0 && threadIdx.x == 0) *ticket = 0;
  const int row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int nrows = E + (gw ? 1 : 0);
  if (row >= nrows) return;
  const uint16_t *wr = row < E ? rw + (size_t)row * H : gw;
  const int nch = H >> 3;
  for (int t0 = 0; t0 < T; t0 += ROUTER_TT) {
    float acc[ROUTER_TT];
#pragma unroll
    for (int i = 0; i < ROUTER_TT; ++i) acc[i] = 0.0f;
    for (int c = lane; c < nch; c += 64) {
      u32x4 wv = *(const u32x4 *)(wr + (size_t)c * 8);
      float wf[8];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        wf[2 * q] = __uint_as_float(wv[q] << 16);
        wf[2 * q + 1] = __uint_as_float(wv[q] & 0xFFFF0000u);
      }
#pragma unroll
      for (int i = 0; i < ROUTER_TT; ++i) {
        if (t0 + i < T) {
          u32x4 xv = *(const u32x4 *)(x + (size_t)(t0 + i) * H + (size_t)c * 8);
          float a = acc[i];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            a = __builtin_fmaf(__uint_as_float(xv[q] << 16), wf[2 * q], a);
            a = __builtin_fmaf(__uint_as_float(xv[q] & 0xFFFF0000u), wf[2 * q + 1], a);
          }
          acc[i] = a;
        }
      }
    }
#pragma unroll
    for (int i = 0; i < ROUTER_TT; ++i) {
      float v = acc[i];
#pragma unroll
      for (int m = 32; m >= 1; m >>= 1) v = v + __shfl_xor(v, m, 64);
      acc[i] = v;
    }
    if (lane == 0) {
#pragma unroll
      for (int i = 0; i < ROUTER_TT; ++i) {
        int t = t0 + i;
        if (t < T) {
          if (row < E)
            logits[(size_t)t * E + row] = bias ? acc[i] + bias[row] : acc[i];
          else
            sg_logit[t] = acc[i];
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Top-k + weights + shared gate + the MFMA-order copy of x.  One wave per
// token.  Lane l holds logits l, l+64, ...; each of the k rounds takes the
// lane-local best (strict >, ascending index), then a wave max of the
// order-preserving key and a wave min of the index among lanes holding that
// key (value descending, index ascending: the CPU oracle's rule).
//
// With `ds` set (T <= 64), the last block to finish also runs the dispatch:
// per-expert 64-bit token masks in LDS (order-free atomic OR), counts, an
// exclusive scan, the tile list, perm / inv / ptok, and it zeroes the
// combine arrival counters.
// ---------------------------------------------------------------------------
constexpr int TOPK_MAXV = 16;  // E <= 1024

__device__ void dispatch_small_block(const int32_t *__restrict__ idx, int T, int k, int E,
                                     int has_shared, const DispatchOut &ds);

__global__ __launch_bounds__(256) void k_topk(const float *__restrict__ logits,
                                              const float *__restrict__ sg_logit,
                                              int has_gate, const uint16_t *__restrict__ x,
                                              int32_t *__restrict__ topk_idx,
                                              float *__restrict__ topk_w,
                                              float *__restrict__ sgate,
                                              uint16_t *__restrict__ xperm, int T, int E,
                                              int k, int H, int has_shared, DispatchOut ds,
                                              int fused) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (t < T) {
    const float *lr = logits + (size_t)t * E;
    uint32_t key[TOPK_MAXV];
#pragma unroll
    for (int i = 0; i < TOPK_MAXV; ++i) {
      int e = lane + 64 * i;
      key[i] = e < E ? ordered_key(lr[e]) : 0u;  // 0: below every finite key
    }
    uint32_t taken = 0;
    int seli = 0;
    for (int j = 0; j < k; ++j) {
      uint32_t bk = 0;
      int bi = 0x7FFFFFFF;
#pragma unroll
      for (int i = 0; i < TOPK_MAXV; ++i) {
        const int e = lane + 64 * i;
        if (e < E && !(taken & (1u << i)) && (bi == 0x7FFFFFFF || key[i] > bk)) {
          bk = key[i];
          bi = e;
        }
      }
      const uint32_t wk = wave_max_u32(bk);
      const int wi = (int)wave_min_u32(bk == wk ? (uint32_t)bi : 0xFFFFFFFFu);
      if ((wi & 63) == lane) taken |= 1u << (wi >> 6);
      if (lane == j) seli = wi;
    }
    // weights: exp(l_j - l_0) / sum_j, sum in slot order
    const float lmax = lr[__builtin_amdgcn_readfirstlane(seli)];
    const float p = lane < k ? expf(lr[seli] - lmax) : 0.0f;
    float sum = 0.0f;
    for (int j = 0; j < k; ++j) sum += __shfl(p, j, 64);
    if (lane < k) {
      topk_idx[(size_t)t * k + lane] = seli;
      topk_w[(size_t)t * k + lane] = p / sum;
    }
    if (lane == 0) sgate[t] = has_gate ? 1.0f / (1.0f + expf(-sg_logit[t])) : 1.0f;
    // MFMA-order copy: 32-element blocks, position 8*j+e <- k = 4*e+j
    if (xperm) {
      const uint16_t *xr = x + (size_t)t * H;
      uint16_t *xo = xperm + (size_t)t * H;
      for (int b = lane; b < (H >> 5); b += 64) {
        const u32x4 *src = (const u32x4 *)(xr + b * 32);
        u32x4 s0 = src[0], s1 = src[1], s2 = src[2], s3 = src[3];
        uint32_t in[16] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3],
                           s2[0], s2[1], s2[2], s2[3], s3[0], s3[1], s3[2], s3[3]};
        uint32_t out[16];
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int e2 = 0; e2 < 4; ++e2) {
            // positions 8j+2e2 and 8j+2e2+1 hold k = 8*e2+j and 8*e2+4+j
            int ka = 8 * e2 + j, kb = ka + 4;
            uint32_t lo = (in[ka >> 1] >> (16 * (ka & 1))) & 0xFFFFu;
            uint32_t hi = (in[kb >> 1] >> (16 * (kb & 1))) & 0xFFFFu;
            out[4 * j + e2] = lo | (hi << 16);
          }
        u32x4 *dst = (u32x4 *)(xo + b * 32);
        dst[0] = u32x4{out[0], out[1], out[2], out[3]};
        dst[1] = u32x4{out[4], out[5], out[6], out[7]};
        dst[2] = u32x4{out[8], out[9], out[10], out[11]};
        dst[3] = u32x4{out[12], out[13], out[14], out[15]};
      }
    }
  }
  if (!fused) return;
  // ---- last block runs the dispatch -------------------------------------
  __shared__ int is_last;
  __syncthreads();
  if (threadIdx.x == 0) {
    __threadfence();
    const int ticket = atomicAdd(ds.ticket, 1);
    is_last = ticket == (int)gridDim.x - 1;
  }
  __syncthreads();
  if (!is_last) return;
  __threadfence();
  if (threadIdx.x == 0) atomicExch(ds.ticket, 0);
  dispatch_small_block(topk_idx, T, k, E, has_shared, ds);
}

// 256 threads, T <= 64.
__device__ void dispatch_small_block(const int32_t *__restrict__ idx, int T, int k, int E,
                                     int has_shared, const DispatchOut &ds) {
  __shared__ unsigned long long mask[1024];
  __shared__ int scan_c[256], scan_t[256];
  __shared__ int off_lds[1024];
  const int tid = threadIdx.x;
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
    t_loc += (c + SMALL_MT - 1) / SMALL_MT;
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
    for (int m0 = 0; m0 < c; m0 += SMALL_MT)
      ds.tiles[tile++] = make_int4(e, off_e + m0, min(SMALL_MT, c - m0), m0);
    off_e += c;
  }
  const int routed_tiles = scan_t[255];
  if (tid == 0) ds.offsets[E] = scan_c[255];
  const int nsh = has_shared ? (T + SMALL_MT - 1) / SMALL_MT : 0;
  if (tid < nsh)
    ds.tiles[routed_tiles + tid] =
        make_int4(E, tid * SMALL_MT, min(SMALL_MT, T - tid * SMALL_MT), tid * SMALL_MT);
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
  for (int i = tid; i < ds.n_cnt; i += 256) ds.cnt[i] = 0;
}

hipError_t launch_router(const void *x, const void *rw, const float *bias, const void *gw,
                         float *logits, float *sg_logit, int32_t *ticket, int T, int H, int E,
                         hipStream_t s) {
  if (T == 0) return hipSuccess;
  int rows = E + (gw ? 1 : 0);
  k_router_logits<<<(rows + 3) / 4, 256, 0, s>>>((const uint16_t *)x, (const uint16_t *)rw,
                                                 bias, (const uint16_t *)gw, logits,
                                                 sg_logit, ticket, T, H, E);
  return hipGetLastError();
}

hipError_t launch_topk(const float *logits, const float *sg_logit, int has_gate,
                       const void *x, int32_t *idx, float *w, float *sg, void *xperm, int T,
                       int E, int k, int H, int has_shared, const DispatchOut *fused,
                       hipStream_t s) {
  if (T == 0) return hipSuccess;
  DispatchOut ds;
  memset(&ds, 0, sizeof ds);
  if (fused) ds = *fused;
  k_topk<<<(T + 3) / 4, 256, 0, s>>>(logits, sg_logit, has_gate, (const uint16_t *)x, idx, w,
                                     sg, (uint16_t *)xperm, T, E, k, H, has_shared, ds,
                                     fused ? 1 : 0);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Dispatch.
//  count: one wave per 64-token chunk.  mask[e] gets bit (t - t0) for every
//         token of the chunk that selected e (64-bit LDS OR: order-free);
//         the rank of (t, j) inside the chunk is popcount of the lower bits.
//  scan:  one block: per-expert prefix over chunks, exclusive scan over
//         experts, and the expert tile list for the grouped kernels.
//  place: pos = chunk_base[c][e] + rank; perm[pos] = t*k+j; inv[t*k+j] = pos.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64) void k_dispatch_count(const int32_t *__restrict__ idx,
                                                       int T, int k, int E,
                                                       int32_t *__restrict__ chunk_counts,
                                                       int32_t *__restrict__ rank) {
  extern __shared__ unsigned long long mask[];
  const int lane = threadIdx.x, c = blockIdx.x;
  for (int e = lane; e < E; e += 64) mask[e] = 0ull;
  __syncthreads();
  const int t = c * 64 + lane;
  if (t < T)
    for (int j = 0; j < k; ++j) atomicOr(&mask[idx[(size_t)t * k + j]], 1ull << lane);
  __syncthreads();
  if (t < T) {
    unsigned long long below = (lane == 0) ? 0ull : ((~0ull) >> (64 - lane));
    for (int j = 0; j < k; ++j) {
      int e = idx[(size_t)t * k + j];
      rank[(size_t)t * k + j] = __popcll(mask[e] & below);
    }
  }
  for (int e = lane; e < E; e += 64) chunk_counts[(size_t)c * E + e] = __popcll(mask[e]);
}

// blockDim = 1024 >= E.  Also emits the tile list: for each expert with
// tokens, ceil(count / mt) tiles (expert, first row), experts ascending,
// then ceil(T / mt) shared-expert tiles (expert id E) when has_shared.
__global__ __launch_bounds__(1024) void k_dispatch_scan(int32_t *__restrict__ chunk_counts,
                                                        int nchunks, int E, int T, int mt,
                                                        int has_shared,
                                                        DispatchOut ds) {
  __shared__ int32_t sc[1024];
  __shared__ int32_t st[1024];
  const int e = threadIdx.x;
  int total = 0;
  if (e < E) {
    for (int c = 0; c < nchunks; ++c) {
      int v = chunk_counts[(size_t)c * E + e];
      chunk_counts[(size_t)c * E + e] = total;  // exclusive within expert
      total += v;
    }
  }
  int ntile = (e < E) ? (total + mt - 1) / mt : 0;
  sc[e] = e < E ? total : 0;
  st[e] = ntile;
  __syncthreads();
  // Hillis-Steele inclusive scans over 1024 entries (integers: exact)
  for (int off = 1; off < 1024; off <<= 1) {
    int a = e >= off ? sc[e - off] : 0;
    int b = e >= off ? st[e - off] : 0;
    __syncthreads();
    sc[e] += a;
    st[e] += b;
    __syncthreads();
  }
  int base = sc[e] - (e < E ? total : 0);
  int tbase = st[e] - ntile;
  if (e < E) {
    ds.counts[e] = total;
    ds.offsets[e] = base;
    for (int c = 0; c < nchunks; ++c) chunk_counts[(size_t)c * E + e] += base;
    if (ds.tiles)
      for (int i = 0; i < ntile; ++i)
        ds.tiles[tbase + i] = make_int4(e, base + i * mt, min(mt, total - i * mt), i * mt);
  }
  if (e == 0) ds.offsets[E] = sc[1023];
  __syncthreads();
  const int routed_tiles = st[1023];
  const int nsh = has_shared ? (T + mt - 1) / mt : 0;
  if (ds.tiles)
    for (int i = e; i < nsh; i += blockDim.x)
      ds.tiles[routed_tiles + i] = make_int4(E, i * mt, min(mt, T - i * mt), i * mt);
  if (e == 0 && ds.n_tiles) *ds.n_tiles = routed_tiles + nsh;
}

__global__ void k_dispatch_place(const int32_t *__restrict__ idx,
                                 const int32_t *__restrict__ rank,
                                 const int32_t *__restrict__ chunk_base, int T, int k, int E,
                                 DispatchOut ds) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  for (int c = i; c < ds.n_cnt; c += gridDim.x * blockDim.x) ds.cnt[c] = 0;
  if (i >= T * k) return;
  const int t = i / k, c = t >> 6;
  const int e = idx[i];
  const int pos = chunk_base[(size_t)c * E + e] + rank[i];
  ds.perm[pos] = i;
  if (ds.inv) ds.inv[i] = pos;
  if (ds.ptok) ds.ptok[pos] = t;
}

hipError_t launch_dispatch(const int32_t *idx, int T, int k, int E, int mt, int has_shared,
                           int32_t *chunk_counts, int32_t *rank, const DispatchOut &ds,
                           hipStream_t s) {
  int nchunks = (T + 63) / 64;
  if (T > 0) {
    k_dispatch_count<<<nchunks, 64, sizeof(unsigned long long) * E, s>>>(idx, T, k, E,
                                                                         chunk_counts, rank);
  }
  k_dispatch_scan<<<1, 1024, 0, s>>>(chunk_counts, nchunks, E, T, mt, has_shared, ds);
  if (T > 0) {
    int n = T * k;
    k_dispatch_place<<<(n + 255) / 256, 256, 0, s>>>(idx, rank, chunk_counts, T, k, E, ds);
  }
  return hipGetLastError();
}


// ---------------------------------------------------------------------------
// Combine: y[t] = sum_j w[t][j] * o[inv[t*k+j]] + g_s[t] * o[T*k + t]
// (+ residual), in slot order with fp32 fma, bf16 out.  One thread per 4
// columns.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_combine(const float *__restrict__ o,
                                                 const int32_t *__restrict__ inv,
                                                 const float *__restrict__ w,
                                                 const float *__restrict__ sg, int has_shared,
                                                 const uint16_t *__restrict__ resid,
                                                 uint16_t *__restrict__ y, int T, int k, int H) {
  const int per_tok = H >> 2;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= T * per_tok) return;
  const int t = i / per_tok, h0 = (i % per_tok) * 4;
  int pos[32];
  float wj[32];
#pragma unroll
  for (int j = 0; j < 32; ++j)
    if (j < k) {
      pos[j] = inv[(size_t)t * k + j];
      wj[j] = w[(size_t)t * k + j];
    }
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < 32; ++j)
    if (j < k) {
      const f32x4 v = *(const f32x4 *)(o + (size_t)pos[j] * H + h0);
#pragma unroll
      for (int q = 0; q < 4; ++q) acc[q] = __builtin_fmaf(wj[j], v[q], acc[q]);
    }
  if (has_shared) {
    const float g = sg[t];
    const f32x4 v = *(const f32x4 *)(o + ((size_t)T * k + t) * H + h0);
#pragma unroll
    for (int q = 0; q < 4; ++q) acc[q] = __builtin_fmaf(g, v[q], acc[q]);
  }
  if (resid) {
    const uint2 r = *(const uint2 *)(resid + (size_t)t * H + h0);
    acc[0] += __uint_as_float(r.x << 16);
    acc[1] += __uint_as_float(r.x & 0xFFFF0000u);
    acc[2] += __uint_as_float(r.y << 16);
    acc[3] += __uint_as_float(r.y & 0xFFFF0000u);
  }
  uint2 out;
  out.x = (uint32_t)f32_to_bf16(acc[0]) | ((uint32_t)f32_to_bf16(acc[1]) << 16);
  out.y = (uint32_t)f32_to_bf16(acc[2]) | ((uint32_t)f32_to_bf16(acc[3]) << 16);
  *(uint2 *)(y + (size_t)t * H + h0) = out;
}

hipError_t launch_combine(const float *o, const int32_t *inv, const float *w, const float *sg,
                          int has_shared, const void *resid, void *y, int T, int k, int H,
                          hipStream_t s) {
  if (T == 0) return hipSuccess;
  const int n = T * (H / 4);
  k_combine<<<(n + 255) / 256, 256, 0, s>>>(o, inv, w, sg, has_shared, (const uint16_t *)resid,
                                            (uint16_t *)y, T, k, H);
  return hipGetLastError();
}
