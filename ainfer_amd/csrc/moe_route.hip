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

#include <type_traits>

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
// RMSNorm: one 256-thread block per row; fp64 sum of squares as a
// lane-strided + pairwise tree (the shape of RMSNormW's N = 5120 form,
// tools/cmdlist/kernels.cpp:94-113), whose float mean rms_mean_f proves equal
// to the reference's sequential order, with a sequential re-sum for the rows
// where it cannot; fp32 normalise, bf16 out.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_rmsnorm(const uint16_t *__restrict__ x,
                                                 const uint16_t *__restrict__ w, int mode,
                                                 float eps, uint16_t *__restrict__ y, int H) {
  __shared__ double ps[256];
  __shared__ int pe[256];
  const int t = blockIdx.x, lid = threadIdx.x;
  const uint16_t *xr = x + (size_t)t * H;
  double ss = 0.0;
  int emin = 0x7FFF;
  for (int j = lid; j < H; j += 256) {
    const uint16_t u = xr[j];
    double v = (double)bf16_to_f32(u);
    ss += v * v;
    emin = min(emin, bf16_qexp(u));
  }
  ps[lid] = ss;
  pe[lid] = emin;
  __syncthreads();
  for (int st = 128; st > 0; st >>= 1) {
    if (lid < st) {
      ps[lid] += ps[lid + st];
      pe[lid] = min(pe[lid], pe[lid + st]);
    }
    __syncthreads();
  }
  float mean;
  if (!rms_mean_f(ps[0], pe[0], H, mean)) {  // block-uniform; see rms_mean_f
    __syncthreads();
    if (lid == 0) ps[0] = row_sumsq_seq(xr, H);
    __syncthreads();
    mean = (float)(ps[0] / H);
  }
  float inv = 1.0f / sqrtf(mean + eps);
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

// The same for rows of 16-byte chunks (H % 8 == 0, H <= 2048 * NC, rows
// 16-byte aligned): thread l holds chunks l, l + 256, ... in registers from
// one load to the store; sums as row_rms_inv (DPP wave reductions, then the
// four waves' partials); normalized pairs as norm_pair.  Bit-identical to
// k_rmsnorm (the mean is order-free whenever rms_mean_f accepts it, else
// re-summed in the reference order).
template <int NC>
__global__ __launch_bounds__(256) void k_rmsnorm_v(const uint16_t *__restrict__ x,
                                                   const uint16_t *__restrict__ w, int mode,
                                                   float eps, uint16_t *__restrict__ y, int H) {
  __shared__ double ps[4];
  __shared__ int pe[4];
  const int t = blockIdx.x, lid = threadIdx.x, lane = lid & 63, wv = lid >> 6;
  const uint16_t *xr = x + (size_t)t * H;
  const int nch = H >> 3;
  u32x4 xv[NC], nv[NC];
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int c = min(lid + 256 * i, nch - 1);
    xv[i] = *(const u32x4 *)(xr + 8 * c);
    nv[i] = w ? *(const u32x4 *)(w + 8 * c) : u32x4{0u, 0u, 0u, 0u};
  }
  double p4[4] = {0.0, 0.0, 0.0, 0.0};
  u16x2_t ek = {0x7F80, 0x7F80};
#pragma unroll
  for (int i = 0; i < NC; ++i)
    if (lid + 256 * i < nch) sumsq_chunk(xv[i], p4, ek);
  const double wtot = wave_sum_f64((p4[0] + p4[1]) + (p4[2] + p4[3]));
  const int wemin = (int)wave_min_u32((uint32_t)ek_emin(ek));
  if (lane == 0) {
    ps[wv] = wtot;
    pe[wv] = wemin;
  }
  __syncthreads();
  const double tot = (ps[0] + ps[1]) + (ps[2] + ps[3]);
  const int emin = min(min(pe[0], pe[1]), min(pe[2], pe[3]));
  float mean;
  if (!rms_mean_f(tot, emin, H, mean)) {  // block-uniform; see rms_mean_f
    __syncthreads();
    if (lid == 0) ps[0] = row_sumsq_seq(xr, H);
    __syncthreads();
    mean = (float)(ps[0] / H);
  }
  const float inv = 1.0f / sqrtf(mean + eps);
  NormIn n;
  n.w = w;
  n.mode = mode;
  n.eps = eps;
  n.on = 1;
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int c = lid + 256 * i;
    if (c < nch) {
      u32x4 o;
#pragma unroll
      for (int q = 0; q < 4; ++q) o[q] = norm_pair(xv[i][q], nv[i][q], inv, n);
      *(u32x4 *)(y + (size_t)t * H + 8 * c) = o;
    }
  }
}

hipError_t launch_rmsnorm(const void *x, const void *w, int mode, float eps, void *y,
                          int T, int H, hipStream_t s) {
  if (T == 0) return hipSuccess;
  const bool vec = (H & 7) == 0 && H <= 8192 && ((uintptr_t)x & 15) == 0 &&
                   ((uintptr_t)y & 15) == 0 && ((uintptr_t)w & 15) == 0;
  const uint16_t *xp = (const uint16_t *)x, *wp = (const uint16_t *)w;
  uint16_t *yp = (uint16_t *)y;
  if (vec && H <= 2048)
    k_rmsnorm_v<1><<<T, 256, 0, s>>>(xp, wp, mode, eps, yp, H);
  else if (vec && H <= 4096)
    k_rmsnorm_v<2><<<T, 256, 0, s>>>(xp, wp, mode, eps, yp, H);
  else if (vec)
    k_rmsnorm_v<4><<<T, 256, 0, s>>>(xp, wp, mode, eps, yp, H);
  else
    k_rmsnorm<<<T, 256, 0, s>>>(xp, wp, mode, eps, yp, H);
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
  if (ticket && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) *ticket = 0;
  const int row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int nrows = E + (gw ? 1 : 0);
  if (row >= nrows) return;
  const uint16_t *wr = row < E ? rw + (size_t)row * H : gw;
  const int nch = H >> 3;
  // blockIdx.y selects ROUTER_TT tokens.  Token rows past T are clamped to
  // T - 1 so that every load is unconditional and the compiler can issue a
  // chunk's ROUTER_TT loads back to back; only the stores are guarded.
  const int t0 = blockIdx.y * ROUTER_TT;
  float acc[ROUTER_TT];
#pragma unroll
  for (int i = 0; i < ROUTER_TT; ++i) acc[i] = 0.0f;
  for (int c = lane; c < nch; c += 64) {
    u32x4 wv = *(const u32x4 *)(wr + (size_t)c * 8);
    u32x4 xv[ROUTER_TT];
#pragma unroll
    for (int i = 0; i < ROUTER_TT; ++i)
      xv[i] = *(const u32x4 *)(x + (size_t)min(t0 + i, T - 1) * H + (size_t)c * 8);
    float wf[8];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      wf[2 * q] = __uint_as_float(wv[q] << 16);
      wf[2 * q + 1] = __uint_as_float(wv[q] & 0xFFFF0000u);
    }
#pragma unroll
    for (int i = 0; i < ROUTER_TT; ++i) {
      float a = acc[i];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        a = __builtin_fmaf(__uint_as_float(xv[i][q] << 16), wf[2 * q], a);
        a = __builtin_fmaf(__uint_as_float(xv[i][q] & 0xFFFF0000u), wf[2 * q + 1], a);
      }
      acc[i] = a;
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

hipError_t launch_router(const void *x, const void *rw, const float *bias, const void *gw,
                         float *logits, float *sg_logit, int32_t *ticket, int T, int H, int E,
                         hipStream_t s) {
  if (T == 0) return hipSuccess;
  int rows = E + (gw ? 1 : 0);
  const dim3 grid((rows + 3) / 4, (T + ROUTER_TT - 1) / ROUTER_TT);
  k_router_logits<<<grid, 256, 0, s>>>((const uint16_t *)x, (const uint16_t *)rw,
                                                 bias, (const uint16_t *)gw, logits,
                                                 sg_logit, ticket, T, H, E);
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

// blockDim = NT >= E (512 when E <= 512: twice the registers per thread
// for the chunk counts).  Also emits the tile list: for each expert with
// tokens, ceil(count / mt) tiles (expert, first row), experts ascending,
// then ceil(T / mt) shared-expert tiles (expert id E) when has_shared.  With
// ds.small_max > 0, an expert with 1..small_max tokens instead gets
// ceil(count / SMALL_MT) tiles in ds.tiles2 (experts ascending), counted in
// ds.n_tiles2.
constexpr int DISPATCH_MAX_CHUNKS = 64;  // 64-token chunks: T <= 4096 per call

template <int NT>
__global__ __launch_bounds__(NT) void k_dispatch_scan(int32_t *__restrict__ chunk_counts,
                                                        int nchunks, int E, int T, int mt,
                                                        int has_shared,
                                                        DispatchOut ds) {
  __shared__ int32_t wsum[2][16];
  const int e = threadIdx.x, lane = e & 63, wv = e >> 6;
  // every chunk count of this expert in registers, all loads in flight at
  // once (nchunks <= DISPATCH_MAX_CHUNKS): one memory round trip, where
  // batches of 16 took four (kernel 9.5 -> 8.1 us at 64 chunks)
  int u[DISPATCH_MAX_CHUNKS];
  int total = 0;
  {
    const int32_t *pc = chunk_counts + min(e, E - 1);  // advanced by one chunk row per load
#pragma unroll
    for (int j = 0; j < DISPATCH_MAX_CHUNKS; ++j) {
      u[j] = e < E && j < nchunks ? *pc : 0;
      pc += E;
    }
  }
#pragma unroll
  for (int j = 0; j < DISPATCH_MAX_CHUNKS; ++j) total += u[j];
  const bool small = ds.small_max > 0 && total > 0 && total <= ds.small_max;
  const int ntile = (ds.tiles && e < E && !small) ? (total + mt - 1) / mt : 0;
  const int nsmall = small ? (total + SMALL_MT - 1) / SMALL_MT : 0;
  // two block scans (integers: exact): token counts, and the big tile count
  // (low 16 bits) with the small tile count (high bits).  Where tiles are
  // written (T * k / mt + E tiles at most, mt = 16 only below 256 tokens)
  // both counts stay below 2^15.
  const int ic = wave_scan_incl(total);
  const int it = wave_scan_incl(ntile | (nsmall << 16));
  if (lane == 63) {
    wsum[0][wv] = ic;
    wsum[1][wv] = it;
  }
  __syncthreads();
  int bc = 0, bt = 0, tc = 0, tt = 0;
#pragma unroll
  for (int w = 0; w < NT / 64; ++w) {
    const int a0 = wsum[0][w], a1 = wsum[1][w];
    bc += w < wv ? a0 : 0;
    bt += w < wv ? a1 : 0;
    tc += a0;
    tt += a1;
  }
  const int base = bc + ic - total;
  const int tb = bt + it - (ntile | (nsmall << 16));
  const int tbase = tb & 0xFFFF, sbase = tb >> 16;
  if (e < E) {
    ds.counts[e] = total;
    ds.offsets[e] = base;
    // chunk_counts[c][e] becomes the first position of chunk c's tokens of e
    int run = base;
#pragma unroll
    for (int j = 0; j < DISPATCH_MAX_CHUNKS; ++j) {
      if (j < nchunks) chunk_counts[(size_t)j * E + e] = run;
      run += u[j];
    }
    if (ds.tiles)
      for (int i = 0; i < ntile; ++i)
        ds.tiles[tbase + i] = make_int4(e, base + i * mt, min(mt, total - i * mt), 0);
    for (int i = 0; i < nsmall; ++i)
      ds.tiles2[sbase + i] = make_int4(e, base + i * SMALL_MT, min(SMALL_MT, total - i * SMALL_MT), 0);
  }
  if (e == 0) ds.offsets[E] = tc;
  if (e == 0 && ds.small_max > 0) *ds.n_tiles2 = tt >> 16;
  const int routed_tiles = tt & 0xFFFF;
  const int nsh = has_shared ? (T + mt - 1) / mt : 0;
  if (ds.tiles)
    for (int i = e; i < nsh; i += blockDim.x)
      ds.tiles[routed_tiles + i] = make_int4(E, i * mt, min(mt, T - i * mt), 0);
  if (e == 0 && ds.n_tiles) *ds.n_tiles = routed_tiles + nsh;
}

__global__ void k_dispatch_place(const int32_t *__restrict__ idx,
                                 const int32_t *__restrict__ rank,
                                 const int32_t *__restrict__ chunk_base, int T, int k, int E,
                                 DispatchOut ds,
                                 const unsigned long long *__restrict__ cmask) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= T * k) return;
  const int t = i / k, c = t >> 6;
  const int e = idx[i];
  // rank of token t among its chunk's tokens of expert e
  const int r = cmask ? __popcll(cmask[(size_t)c * E + e] & ((1ull << (t & 63)) - 1ull)) : rank[i];
  const int pos = chunk_base[(size_t)c * E + e] + r;
  ds.perm[pos] = i;
  if (ds.inv) ds.inv[i] = pos;
  if (ds.ptok) ds.ptok[pos] = t;
}

hipError_t launch_dispatch(const int32_t *idx, int T, int k, int E, int mt, int has_shared,
                           int32_t *chunk_counts, int32_t *rank, const DispatchOut &ds,
                           hipStream_t s, const unsigned long long *cmask) {
  const int nchunks = (T + 63) / 64;
  if (nchunks > DISPATCH_MAX_CHUNKS) return hipErrorInvalidValue;
  if (T > 0 && !cmask) {
    k_dispatch_count<<<nchunks, 64, sizeof(unsigned long long) * E, s>>>(idx, T, k, E,
                                                                         chunk_counts, rank);
  }
  if (E <= 512)
    k_dispatch_scan<512><<<1, 512, 0, s>>>(chunk_counts, nchunks, E, T, mt, has_shared, ds);
  else
    k_dispatch_scan<1024><<<1, 1024, 0, s>>>(chunk_counts, nchunks, E, T, mt, has_shared, ds);
  if (T > 0) {
    int n = T * k;
    k_dispatch_place<<<(n + 255) / 256, 256, 0, s>>>(idx, rank, chunk_counts, T, k, E, ds, cmask);
  }
  return hipGetLastError();
}


// ---------------------------------------------------------------------------
// Combine: y[t] = sum_j w[t][j] * o[inv[t*k+j]] + g_s[t] * o[T*k + t]
// (+ residual), in slot order with fp32 fma, bf16 out.  One thread per CPT
// columns (8: 16-byte loads).
// ---------------------------------------------------------------------------
template <int CPT>
__global__ __launch_bounds__(256) void k_combine(const uint16_t *__restrict__ o,
                                                 const int32_t *__restrict__ inv,
                                                 const float *__restrict__ w,
                                                 const float *__restrict__ sg, int has_shared,
                                                 const uint16_t *__restrict__ resid,
                                                 uint16_t *__restrict__ y, int T, int k, int H,
                                                 const int32_t *__restrict__ err) {
  typedef uint32_t vec_t __attribute__((ext_vector_type(CPT / 2)));
  // grid (T, ceil(H / (CPT * blockDim.x))): the token is uniform, so its
  // slots' positions and weights are scalar loads
  const int t = blockIdx.x, h0 = (blockIdx.y * blockDim.x + threadIdx.x) * CPT;
  if (h0 >= H) return;
  int pos[32];
  float wj[32];
#pragma unroll
  for (int j = 0; j < 32; ++j)
    if (j < k) {
      pos[j] = inv ? inv[(size_t)t * k + j] : t * k + j;  // null: rows in slot order
      wj[j] = w[(size_t)t * k + j];
    }
  float acc[CPT];
#pragma unroll
  for (int q = 0; q < CPT; ++q) acc[q] = 0.0f;
  auto fma_row = [&](float g, const vec_t &rv) {
#pragma unroll
    for (int q = 0; q < CPT / 2; ++q) {
      acc[2 * q] = __builtin_fmaf(g, __uint_as_float(rv[q] << 16), acc[2 * q]);
      acc[2 * q + 1] = __builtin_fmaf(g, __uint_as_float(rv[q] & 0xFFFF0000u), acc[2 * q + 1]);
    }
  };
  // slots in batches of 8: the batch's loads first, then its fmas in slot order
  constexpr int B = 8;
#pragma unroll
  for (int j0 = 0; j0 < 32; j0 += B) {
    if (j0 >= k) break;
    vec_t r[B];
#pragma unroll
    for (int j = 0; j < B; ++j)
      r[j] = __builtin_nontemporal_load((const vec_t *)(o + (size_t)pos[min(j0 + j, k - 1)] * H + h0));
#pragma unroll
    for (int j = 0; j < B; ++j)
      if (j0 + j < k) fma_row(wj[j0 + j], r[j]);
  }
  if (has_shared)
    fma_row(sg[t], __builtin_nontemporal_load((const vec_t *)(o + ((size_t)T * k + t) * H + h0)));
  if (resid) {
    const vec_t rr = *(const vec_t *)(resid + (size_t)t * H + h0);
#pragma unroll
    for (int q = 0; q < CPT / 2; ++q) {
      acc[2 * q] += __uint_as_float(rr[q] << 16);
      acc[2 * q + 1] += __uint_as_float(rr[q] & 0xFFFF0000u);
    }
  }
  vec_t out;
#pragma unroll
  for (int q = 0; q < CPT / 2; ++q)
    out[q] = (uint32_t)f32_to_bf16(acc[2 * q]) | ((uint32_t)f32_to_bf16(acc[2 * q + 1]) << 16);
  // a bounded device wait of this or an earlier call on the workspace ran
  // out: the output is not to be trusted, so it is made NaN (until re-init)
  if (err && *err) {
#pragma unroll
    for (int q = 0; q < CPT / 2; ++q) out[q] = 0x7FC07FC0u;
  }
  *(vec_t *)(y + (size_t)t * H + h0) = out;
}

// Combine with the residual, then the next block's RMSNorm of the row just
// written, so a stack of blocks needs no RMSNorm launch between them (the
// residual add fused into the norm, as tools/norm/norm.cpp:30-61 does with
// FUSED = true).  One block of NT = H / 8 threads (rounded up to whole waves)
// per token: thread l holds chunk l of the row from the combine to the norm,
// with every slot's load of it in flight at once.  Each output element is
// k_combine's arithmetic (slot order fmaf, shared expert, residual, bf16); h
// is k_rmsnorm's on those bf16 values (the fp64 mean is order-free whenever
// rms_mean_f accepts it, else the row is re-summed sequentially from an LDS
// copy).
template <int NT>
__global__ __launch_bounds__(NT) void k_combine_norm(
    const uint16_t *__restrict__ o, const int32_t *__restrict__ inv, const float *__restrict__ w,
    const float *__restrict__ sg, int has_shared, const uint16_t *resid, uint16_t *y, int T,
    int k, int H, const int32_t *__restrict__ err, const uint16_t *__restrict__ nw, int mode,
    float eps, uint16_t *__restrict__ h) {
  constexpr int NWV = NT / 64;
  __shared__ double ps[NWV];
  __shared__ int pe[NWV];
  __shared__ __attribute__((aligned(16))) uint16_t srow[NT * 8];
  const int t = blockIdx.x, lid = threadIdx.x, lane = lid & 63, wv = lid >> 6;
  const int nch = H >> 3;
  const bool live = lid < nch;
  const int c = min(lid, nch - 1);
  const bool bad = err && *err;
  int pos[32];
  float wj[32];
#pragma unroll
  for (int j = 0; j < 32; ++j)
    if (j < k) {
      pos[j] = inv ? inv[(size_t)t * k + j] : t * k + j;
      wj[j] = w[(size_t)t * k + j];
    }
  // loads of up to 16 slots in flight, then their fmas in slot order
  constexpr int B = 16;
  float acc[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) acc[q] = 0.0f;
  auto fma_row = [&](float g, const u32x4 &rv) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      acc[2 * q] = __builtin_fmaf(g, __uint_as_float(rv[q] << 16), acc[2 * q]);
      acc[2 * q + 1] = __builtin_fmaf(g, __uint_as_float(rv[q] & 0xFFFF0000u), acc[2 * q + 1]);
    }
  };
  const u32x4 nv = nw ? *(const u32x4 *)(nw + 8 * c) : u32x4{0u, 0u, 0u, 0u};
  const u32x4 rr = *(const u32x4 *)(resid + (size_t)t * H + 8 * c);
  const u32x4 sv = has_shared ? __builtin_nontemporal_load((const u32x4 *)(o + ((size_t)T * k + t) * H + 8 * c))
                              : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
  for (int j0 = 0; j0 < 32; j0 += B) {
    if (j0 >= k) break;
    u32x4 r[B];
#pragma unroll
    for (int j = 0; j < B; ++j)
      if (j0 + j < k) r[j] = __builtin_nontemporal_load((const u32x4 *)(o + (size_t)pos[j0 + j] * H + 8 * c));
#pragma unroll
    for (int j = 0; j < B; ++j)
      if (j0 + j < k) fma_row(wj[j0 + j], r[j]);
  }
  if (has_shared) fma_row(sg[t], sv);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    acc[2 * q] += __uint_as_float(rr[q] << 16);
    acc[2 * q + 1] += __uint_as_float(rr[q] & 0xFFFF0000u);
  }
  u32x4 yv;
#pragma unroll
  for (int q = 0; q < 4; ++q)
    yv[q] = bad ? 0x7FC07FC0u
                : (uint32_t)f32_to_bf16(acc[2 * q]) | ((uint32_t)f32_to_bf16(acc[2 * q + 1]) << 16);
  // y may alias resid: each chunk is read and then written by one thread only
  if (live) *(u32x4 *)(y + (size_t)t * H + 8 * c) = yv;
  double p4[4] = {0.0, 0.0, 0.0, 0.0};
  u16x2_t ek = {0x7F80, 0x7F80};
  if (live) sumsq_chunk(yv, p4, ek);
  const double wtot = wave_sum_f64((p4[0] + p4[1]) + (p4[2] + p4[3]));
  const int wemin = (int)wave_min_u32((uint32_t)ek_emin(ek));
  if (lane == 0) {
    ps[wv] = wtot;
    pe[wv] = wemin;
  }
  __syncthreads();
  double tot = ps[0];
  int emin = pe[0];
#pragma unroll
  for (int i = 1; i < NWV; ++i) {
    tot += ps[i];
    emin = min(emin, pe[i]);
  }
  float mean;
  if (!rms_mean_f(tot, emin, H, mean)) {  // block-uniform; see rms_mean_f
    if (live) *(u32x4 *)(srow + 8 * c) = yv;
    __syncthreads();
    if (lid == 0) ps[0] = row_sumsq_seq(srow, H);
    __syncthreads();
    mean = (float)(ps[0] / H);
  }
  const float rinv = 1.0f / sqrtf(mean + eps);
  NormIn n;
  n.w = nw;
  n.mode = mode;
  n.eps = eps;
  n.on = 1;
  if (live) {
    u32x4 ov;
#pragma unroll
    for (int q = 0; q < 4; ++q) ov[q] = norm_pair(yv[q], nv[q], rinv, n);
    *(u32x4 *)(h + (size_t)t * H + 8 * c) = ov;
  }
}

hipError_t launch_combine_norm(const uint16_t *o, const int32_t *inv, const float *w,
                               const float *sg, int has_shared, const void *resid, void *y,
                               int T, int k, int H, const int32_t *err, const NormIn &next,
                               void *h, hipStream_t s) {
  if (T == 0) return hipSuccess;
  if (!resid || H % 8 || H > 4096 || k > 32 || ((uintptr_t)resid & 15) || ((uintptr_t)y & 15) ||
      ((uintptr_t)h & 15) || ((uintptr_t)next.w & 15))
    return hipErrorInvalidValue;
  const uint16_t *r = (const uint16_t *)resid, *nw = next.w;
  const int nch = H / 8;
  auto go = [&](auto nt_c) {
    constexpr int NT = decltype(nt_c)::value;
    k_combine_norm<NT><<<T, NT, 0, s>>>(o, inv, w, sg, has_shared, r, (uint16_t *)y, T, k, H, err,
                                        nw, next.mode, next.eps, (uint16_t *)h);
  };
  if (nch <= 64)
    go(std::integral_constant<int, 64>());
  else if (nch <= 128)
    go(std::integral_constant<int, 128>());
  else if (nch <= 256)
    go(std::integral_constant<int, 256>());
  else
    go(std::integral_constant<int, 512>());
  return hipGetLastError();
}

// x in MFMA order and (xsum non-null) its per-128 group sums: one wave per
// token, the copy the routers write beside their logits
__global__ __launch_bounds__(256) void k_xperm(const uint16_t *__restrict__ x,
                                               uint16_t *__restrict__ xperm,
                                               float *__restrict__ xsum, int T, int H) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (t < T) write_xperm(x + (size_t)t * H, xperm, xsum, t, H, lane);
}

hipError_t launch_xperm(const void *x, void *xperm, float *xsum, int T, int H, hipStream_t s) {
  if (T == 0) return hipSuccess;
  k_xperm<<<(T + 3) / 4, 256, 0, s>>>((const uint16_t *)x, (uint16_t *)xperm, xsum, T, H);
  return hipGetLastError();
}

// dst row t * k + j = src row inv[t * k + j] (dispatch position -> slot
// order); rows T * k + t (the shared expert's) copied as they are
__global__ __launch_bounds__(256) void k_gather_rows(const uint16_t *__restrict__ src,
                                                     const int32_t *__restrict__ inv,
                                                     uint16_t *__restrict__ dst, int T, int k,
                                                     int H) {
  const int r = blockIdx.x;
  const size_t from = r < T * k ? (size_t)inv[r] : (size_t)r;
  const u32x4 *a = (const u32x4 *)(src + from * H);
  u32x4 *b = (u32x4 *)(dst + (size_t)r * H);
  for (int i = threadIdx.x; i < H / 8; i += blockDim.x) b[i] = a[i];
}

hipError_t launch_gather_rows(const void *src, const int32_t *inv, void *dst, int T, int k,
                              int H, int has_shared, hipStream_t s) {
  const int rows = T * k + (has_shared ? T : 0);
  if (rows == 0) return hipSuccess;
  k_gather_rows<<<rows, 256, 0, s>>>((const uint16_t *)src, inv, (uint16_t *)dst, T, k, H);
  return hipGetLastError();
}

hipError_t launch_combine(const uint16_t *o, const int32_t *inv, const float *w, const float *sg,
                          int has_shared, const void *resid, void *y, int T, int k, int H,
                          const int32_t *err, hipStream_t s) {
  if (T == 0) return hipSuccess;
  // few tokens: 64-thread blocks, so the layer's columns spread over more CUs
  const int nt = T <= 64 ? 64 : 256;
  if (H % 8 == 0)
    k_combine<8><<<dim3(T, (H / 8 + nt - 1) / nt), nt, 0, s>>>(
        o, inv, w, sg, has_shared, (const uint16_t *)resid, (uint16_t *)y, T, k, H, err);
  else
    k_combine<4><<<dim3(T, (H / 4 + nt - 1) / nt), nt, 0, s>>>(
        o, inv, w, sg, has_shared, (const uint16_t *)resid, (uint16_t *)y, T, k, H, err);
  return hipGetLastError();
}
