// moe_router.hip - router for gfx950: MFMA logits, exact candidate refine,
// top-k, renormalised weights, sigmoid shared gate.
//
// The top-k must equal, bit for bit, the top-k of the fp32 logits computed in
// the lane-strided chunk order (include/ainfer_moe.h).  Computing that order
// for all E experts is a latency-bound VALU job, so the router runs in two
// kernels:
//
//  k_router_mfma: approximate logits on bf16 MFMA (products exact, fp32
//    accumulation in the hardware's order) plus the 2-norm of every router
//    weight row.
//  k_select: one wave per token.  With L_k the k-th largest approximate
//    logit and d >= |approx - exact| + |canonical - exact| for every expert,
//    any expert whose canonical logit can reach the canonical top-k has
//    approx >= L_k - 2d (the top-k experts by approx all have canonical >=
//    L_k - d).  Those candidates are recomputed in the canonical order and
//    the top-k is taken among them: the result equals the top-k over all E
//    canonical logits.  d is a rigorous fp32 summation bound: for n products
//    accumulated with one rounding each (to nearest or toward zero),
//    |error| <= n * 2^-23 * sum|x_i w_i| <= n * 2^-23 * ||x|| * ||w_e||
//    (Cauchy-Schwarz), taken for both paths, plus margins for the bias
//    addition and for denormal flushing.  When many logits tie, every expert
//    becomes a candidate and the same code recomputes all of them.
//
// The dispatch for T <= 64 runs in k_select's last block (dispatch_small_block,
// moe_dispatch.h).
#include <string.h>

#include "moe_common.h"
#include "moe_dispatch.h"
#include "moe_topk.h"
#include "moe_internal.h"

#ifdef AINFER_DECODE_TRACE
__device__ unsigned long long g_strace[4096][8];
#define STRACE(I) \
  if ((threadIdx.x & 63) == 0 && (!COOP || threadIdx.x == 0) && t < 4096) \
  g_strace[t][I] = __builtin_amdgcn_s_memrealtime()
extern "C" int ainfer_debug_strace(void *host) {
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(g_strace), sizeof(g_strace)) == hipSuccess ? 0 : -1;
}
#else
#define STRACE(I)
#endif

namespace {

// ---------------------------------------------------------------------------
// Approximate logits.  Block = NW waves over one (16-expert, 16*MS-token)
// tile; wave w takes k-slice [w*H/NW, (w+1)*H/NW) in 32-wide MFMA steps.
// Lane l: expert row l%16, k offset 8*(l/16) inside each step (A and B use
// the same k mapping, so both operands load 16 contiguous bytes).
// ---------------------------------------------------------------------------
template <int MS>
__global__ __launch_bounds__(1024) void k_router_mfma(const uint16_t *__restrict__ x,
                                                      const uint16_t *__restrict__ rw,
                                                      const float *__restrict__ bias,
                                                      float *__restrict__ approx,
                                                      float *__restrict__ wnorm,
                                                      int32_t *__restrict__ ticket, int T, int H,
                                                      int E, int NW) {
  extern __shared__ float red[];  // [NW][MS*256] partial logits, then [NW][16] norms
  // the last-block counter of the following k_select launch starts at 0
  if (ticket && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) *ticket = 0;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int n = lane & 15, q = lane >> 4;
  const int e0 = blockIdx.x * 16, t0 = blockIdx.y * 16 * MS;
  const int e = min(e0 + n, E - 1);
  const int steps = H / (32 * NW);  // 32-wide k-steps of this wave
  const int kbase = wave * steps * 32;
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(x, (uint32_t)T * (uint32_t)H * 2u);
  f32x4 acc[MS];
#pragma unroll
  for (int ms = 0; ms < MS; ++ms) acc[ms] = f32x4{0.f, 0.f, 0.f, 0.f};
  float ss = 0.0f;
  const uint16_t *wrow = rw + (size_t)e * H + kbase + 8 * q;
  uint32_t xoff[MS];
#pragma unroll
  for (int ms = 0; ms < MS; ++ms) {
    const int t = t0 + 16 * ms + n;
    xoff[ms] = t < T ? ((uint32_t)t * (uint32_t)H + (uint32_t)(kbase + 8 * q)) * 2u : BUF_OOB;
  }
  for (int s0 = 0; s0 < steps; s0 += 4) {
    u32x4 wv[4], xv[MS][4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int ss_ = min(s0 + s, steps - 1);
      wv[s] = *(const u32x4 *)(wrow + 32 * ss_);
#pragma unroll
      for (int ms = 0; ms < MS; ++ms)
        xv[ms][s] = buf_load16(xr, xoff[ms] == BUF_OOB ? BUF_OOB : xoff[ms] + 64u * ss_);
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      if (s0 + s < steps) {
#pragma unroll
        for (int ms = 0; ms < MS; ++ms) acc[ms] = mfma_bf16_16x16x32(xv[ms][s], wv[s], acc[ms]);
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const float lo = __uint_as_float(wv[s][d] << 16), hi = __uint_as_float(wv[s][d] & 0xFFFF0000u);
          ss = __builtin_fmaf(lo, lo, ss);
          ss = __builtin_fmaf(hi, hi, ss);
        }
      }
    }
  }
  // partial logits: lane (q, n) holds tokens 4q+r of each m-subtile, expert n
#pragma unroll
  for (int ms = 0; ms < MS; ++ms)
#pragma unroll
    for (int r = 0; r < 4; ++r) red[wave * (MS * 256) + ms * 256 + (4 * q + r) * 16 + n] = acc[ms][r];
  ss += __shfl_xor(ss, 16, 64);
  ss += __shfl_xor(ss, 32, 64);
  float *nred = red + NW * MS * 256;
  if (q == 0) nred[wave * 16 + n] = ss;
  __syncthreads();
  for (int idx = threadIdx.x; idx < MS * 256; idx += blockDim.x) {
    const int ms = idx >> 8, cell = idx & 255;
    const int t = t0 + 16 * ms + (cell >> 4), ee = e0 + (cell & 15);
    if (t >= T || ee >= E) continue;
    float v = 0.0f;
    for (int w = 0; w < NW; ++w) v += red[w * (MS * 256) + idx];
    approx[(size_t)t * E + ee] = bias ? v + bias[ee] : v;
  }
  if (blockIdx.y == 0 && threadIdx.x < 16 && e0 + (int)threadIdx.x < E) {
    float v = 0.0f;
    for (int w = 0; w < NW; ++w) v += nred[w * 16 + threadIdx.x];
    wnorm[e0 + threadIdx.x] = sqrtf(v);
  }
}

// ---------------------------------------------------------------------------
// canonical dot: x in registers (lane l holds chunks l, l+64, ...), one
// router row w; sequential fma in chunk order, then the xor butterfly.
// ---------------------------------------------------------------------------
template <int CH>
__device__ __forceinline__ float canon_dot(const u32x4 (&xc)[CH], const uint16_t *w, int lane,
                                           int nch) {
  u32x4 wv[CH];
#pragma unroll
  for (int j = 0; j < CH; ++j) {
    const int c = min(lane + 64 * j, nch - 1);
    wv[j] = *(const u32x4 *)(w + (size_t)c * 8);
  }
  float acc = 0.0f;
#pragma unroll
  for (int j = 0; j < CH; ++j) {
    if (lane + 64 * j < nch) {
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        acc = __builtin_fmaf(__uint_as_float(xc[j][d] << 16), __uint_as_float(wv[j][d] << 16), acc);
        acc = __builtin_fmaf(__uint_as_float(xc[j][d] & 0xFFFF0000u),
                             __uint_as_float(wv[j][d] & 0xFFFF0000u), acc);
      }
    }
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) acc = acc + __shfl_xor(acc, m, 64);
  return acc;
}

// NB canonical dots at once (loads of all rows issued before any math);
// rows past nrows repeat the last row and their results are ignored.
template <int CH, int NB>
__device__ __forceinline__ void canon_dot_batch(const u32x4 (&xc)[CH], const uint16_t *const (&w)[NB],
                                                int lane, int nch, float (&out)[NB]) {
  u32x4 wv[NB][CH];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const int c = min(lane + 64 * j, nch - 1);
      wv[b][j] = *(const u32x4 *)(w[b] + (size_t)c * 8);
    }
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      if (lane + 64 * j < nch) {
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          acc = __builtin_fmaf(__uint_as_float(xc[j][d] << 16), __uint_as_float(wv[b][j][d] << 16), acc);
          acc = __builtin_fmaf(__uint_as_float(xc[j][d] & 0xFFFF0000u),
                               __uint_as_float(wv[b][j][d] & 0xFFFF0000u), acc);
        }
      }
    }
    out[b] = acc;
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1)
#pragma unroll
    for (int b = 0; b < NB; ++b) out[b] = out[b] + __shfl_xor(out[b], m, 64);
}


constexpr int SEL_WAVES = 4;
#ifndef SEL_NB
#define SEL_NB 4  // candidate rows whose loads are issued together
#endif

// EXACT: `approx` already holds the canonical logits (k_router_logits) and
// `sgl` the canonical shared-gate logits; the refine is skipped.
// COOP (T < GEMM_MIN_T, where one wave per token leaves most of the chip
// idle and a token's latency is the kernel's): one token per workgroup.
// Wave 0 takes the approximate top-k and the candidate list, wave 1 writes
// the MFMA-order copy of x, wave 2 the shared-gate dot, and the candidates'
// canonical dots are shared by all waves (c3 T=64: the dots were 13 of 25 us
// per token).
template <int NV, int CH, bool EXACT, bool COOP = false>
__global__ __launch_bounds__(256) void k_select(const float *__restrict__ approx,
                                                const float *__restrict__ sgl,
                                                const float *__restrict__ wnorm,
                                                const uint16_t *__restrict__ x,
                                                const uint16_t *__restrict__ rw,
                                                const float *__restrict__ bias,
                                                const uint16_t *__restrict__ gw,
                                                int32_t *__restrict__ topk_idx,
                                                float *__restrict__ topk_w,
                                                float *__restrict__ sgate,
                                                uint16_t *__restrict__ xperm,
                                                float *__restrict__ xsum, int T, int E,
                                                int k, int H, int has_shared, DispatchOut ds,
                                                int fused, unsigned long long *cmask,
                                                int32_t *ccount) {
  // candidate lists (fast path only)
  __shared__ int cl[SEL_WAVES][EXACT ? 1 : 1024];
  __shared__ float cv[SEL_WAVES][EXACT ? 1 : 1024];
  __shared__ uint64_t s_cand[SEL_WAVES][64];
  __shared__ uint64_t s_sel[SEL_WAVES][16];
  __shared__ int s_nc;
  __shared__ float s_sgv;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int t = COOP ? (int)blockIdx.x : (int)blockIdx.x * SEL_WAVES + wave;
  const int sw = COOP ? 0 : wave;  // this wave's LDS lists
  const bool lead = !COOP || wave == 0;
  static_assert(!(COOP && EXACT), "the cooperative form refines approximate logits");
  if (t < T) {
    // the MFMA-order copy of x (and its group sums) does not depend on the
    // routing: written first, its latency hides under the selection
    STRACE(0);
    if (xperm && (!COOP || wave == 1)) write_xperm(x + (size_t)t * H, xperm, xsum, t, H, lane);
    STRACE(1);
    const float *ar = approx + (size_t)t * E;
    // ---- k-th largest approximate logit -------------------------------
    uint32_t key[NV];
    float wn = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      if (!lead) break;
      const int e = lane + 64 * i;
      const float v = ar[min(e, E - 1)];  // unconditional: loads issue together
      key[i] = e < E ? ordered_key(v) : 0u;
      if (!EXACT) wn = fmaxf(wn, e < E ? wnorm[min(e, E - 1)] : 0.0f);
    }
    int seli = 0;
    uint32_t selk = 0u;
    if (lead) wave_topk_fast<NV>(key, E, k, lane, seli, selk, s_cand[sw], s_sel[sw]);
    STRACE(2);
    const uint32_t kth = (uint32_t)__shfl((int)selk, k - 1, 64);
    float selv = 0.0f, sgv = 0.0f;
    const uint16_t *xrow = x + (size_t)t * H;
    if (EXACT) {
      // canonical logits already: the picks above are the top-k
      if (lane < k) selv = ar[seli];
      if (gw) sgv = sgl[t];
    } else {
      // ---- x row in registers (canonical chunk layout) and its norm ------
      const int nch = H >> 3;
      u32x4 xc[CH];
      float xs = 0.0f;
#pragma unroll
      for (int j = 0; j < CH; ++j) {
        const int c = min(lane + 64 * j, nch - 1);
        xc[j] = *(const u32x4 *)(xrow + (size_t)c * 8);
        if (lane + 64 * j < nch) {
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            const float lo = __uint_as_float(xc[j][d] << 16), hi = __uint_as_float(xc[j][d] & 0xFFFF0000u);
            xs = __builtin_fmaf(lo, lo, xs);
            xs = __builtin_fmaf(hi, hi, xs);
          }
        }
      }
      for (int m = 32; m >= 1; m >>= 1) xs += __shfl_xor(xs, m, 64);
      if (COOP && wave == 2 && gw) s_sgv = canon_dot<CH>(xc, gw, lane, nch);
      for (int m = 32; m >= 1; m >>= 1) wn = fmaxf(wn, __shfl_xor(wn, m, 64));
      // ---- candidate threshold --------------------------------------------
      const float lk = key_to_float(kth);
      const float nrm = sqrtf(xs) * wn * 1.0625f;
      const float d = 2.0f * (float)(H + 64) * 0x1p-23f * nrm;  // |approx - canonical|
      const float thr = lk - 2.0f * d - 0x1p-21f * (fabsf(lk) + 2.0f * d) - 1e-30f * (float)H;
      // ---- candidate list, expert-ascending -------------------------------
      int nc = 0;
      if (lead) {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
          const int e = lane + 64 * i;
          const bool c = e < E && key_to_float(key[i]) >= thr;
          const uint64_t b = __ballot(c);
          if (c) cl[sw][nc + __popcll(b & ((1ull << lane) - 1ull))] = e;
          nc += __popcll(b);
        }
        if (COOP && lane == 0) s_nc = nc;
      }
      __builtin_amdgcn_wave_barrier();
      if (COOP) {
        __syncthreads();
        nc = s_nc;
      }
      STRACE(3);
      // ---- canonical logits of the candidates ------------------------------
      {
        const int cstep = COOP ? SEL_WAVES * SEL_NB : SEL_NB;
        for (int c0 = COOP ? wave * SEL_NB : 0; c0 < nc; c0 += cstep) {
          const uint16_t *rows[SEL_NB];
          int ee[SEL_NB];
#pragma unroll
          for (int b = 0; b < SEL_NB; ++b) {
            ee[b] = cl[sw][min(c0 + b, nc - 1)];
            rows[b] = rw + (size_t)ee[b] * H;
          }
          float v[SEL_NB];
          canon_dot_batch<CH, SEL_NB>(xc, rows, lane, nch, v);
#pragma unroll
          for (int b = 0; b < SEL_NB; ++b)
            if (lane == 0 && c0 + b < nc) cv[sw][c0 + b] = bias ? v[b] + bias[ee[b]] : v[b];
        }
      }
      __builtin_amdgcn_wave_barrier();
      if (COOP) __syncthreads();
      STRACE(4);
      // ---- top-k among candidates (value desc, expert asc) ----------------
      if (!lead) {
        // helper waves are done
      } else if (nc <= 64 && k <= 16) {
        // rank of each candidate = candidates above it (unique composite keys)
        auto comp = [&](int i) {
          return ((uint64_t)ordered_key(cv[sw][i]) << 32) | (uint32_t)~(uint32_t)cl[sw][i];
        };
        const uint64_t mine = lane < nc ? comp(lane) : 0ull;
        int rk = 0;
        for (int j = 0; j < nc; ++j) rk += comp(j) > mine ? 1 : 0;
        if (lane < nc && rk < k) s_sel[sw][rk] = ((uint64_t)(uint32_t)lane << 32) | (uint32_t)cl[sw][lane];
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        if (lane < k) {
          const uint64_t pk = s_sel[sw][lane];
          seli = (int)(uint32_t)pk;
          selv = cv[sw][(int)(pk >> 32)];
        }
      } else {
      uint32_t tmask = 0;  // taken bits per lane slot (nc <= 1024: 16 slots)
      for (int j = 0; j < k; ++j) {
        uint32_t bk = 0;
        int bs = 0x7FFFFFFF;
        for (int i = 0; i < 16 && lane + 64 * i < nc; ++i) {
          const uint32_t kk = ordered_key(cv[sw][lane + 64 * i]);
          if (!(tmask & (1u << i)) && (bs == 0x7FFFFFFF || kk > bk)) {
            bk = kk;
            bs = lane + 64 * i;
          }
        }
        const uint32_t wk = wave_max_u32(bk);
        const int ws = (int)wave_min_u32(bk == wk && bs != 0x7FFFFFFF ? (uint32_t)bs : 0xFFFFFFFFu);
        if ((ws & 63) == lane) tmask |= 1u << (ws >> 6);
        if (lane == j) {
          seli = cl[sw][ws];
          selv = cv[sw][ws];
        }
      }
      }
      STRACE(5);
      if (gw) sgv = COOP ? s_sgv : canon_dot<CH>(xc, gw, lane, nch);
      STRACE(6);
    }
    if (lead) {
      const float vmax = __shfl(selv, 0, 64);
      const float p = lane < k ? expf(selv - vmax) : 0.0f;
      float sum = 0.0f;
      for (int j = 0; j < k; ++j) sum += __shfl(p, j, 64);
      if (lane < k) {
        topk_idx[(size_t)t * k + lane] = seli;
        topk_w[(size_t)t * k + lane] = p / sum;
        // the dispatch's count and token mask of (64-token chunk, expert):
        // a sum and an OR over the chunk's picks, so the order of the
        // atomics does not matter (the counts sit just before the masks)
        if (cmask) {
          const size_t ce = (size_t)(t >> 6) * E + seli;
          atomicOr(cmask + ce, 1ull << (t & 63));
          atomicAdd(ccount + ce, 1);
        }
      }
      // ---- shared gate --------------------------------------------------
      float g = 1.0f;
      if (gw) g = 1.0f / (1.0f + expf(-sgv));
      if (lane == 0) sgate[t] = g;
    }
    STRACE(7);
  }
  if (!fused) return;
  // ---- the last block runs the dispatch ---------------------------------
  __shared__ int is_last;
  __syncthreads();
  if (threadIdx.x == 0) {
    __threadfence();
    is_last = atomicAdd(ds.ticket, 1) == (int)gridDim.x - 1;
  }
  __syncthreads();
  if (!is_last) return;
  __threadfence();
  if (threadIdx.x == 0) atomicExch(ds.ticket, 0);
  dispatch_small_block(topk_idx, T, k, E, has_shared, ds);
}

// Decode routing for T <= 16 in one block, one wave per token: the exact
// top-k of the canonical logits, softmax weights, the shared-expert gate and
// the MFMA-order copy of x; then wave 0 builds the dispatch from the picks
// kept in LDS (tiles of at most DEC_MT tokens).
__device__ __forceinline__ void dispatch_wave(const int *__restrict__ s_idx, int T, int k, int E,
                                              int has_shared, const DispatchOut &ds,
                                              uint32_t *msk, int *off, int lane) {
  for (int e = lane; e < E; e += 64) msk[e] = 0u;
  __builtin_amdgcn_wave_barrier();
  for (int i = lane; i < T * k; i += 64) atomicOr(&msk[s_idx[i]], 1u << (i / k));
  __builtin_amdgcn_wave_barrier();
  // lane owns experts [e0, e1): counts, then one tile per expert with tokens
  const int npl = (E + 63) / 64, e0 = lane * npl, e1 = min(e0 + npl, E);
  int c_loc = 0, t_loc = 0;
  for (int e = e0; e < e1; ++e) {
    const int c = __popc(msk[e]);
    c_loc += c;
    t_loc += (c + DEC_MT - 1) / DEC_MT;
  }
  int c_inc = c_loc, t_inc = t_loc;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int a = __shfl_up(c_inc, d, 64), b = __shfl_up(t_inc, d, 64);
    if (lane >= d) {
      c_inc += a;
      t_inc += b;
    }
  }
  int o = c_inc - c_loc, tb = t_inc - t_loc;
  for (int e = e0; e < e1; ++e) {
    const uint32_t m = msk[e];
    const int c = __popc(m);
    ds.counts[e] = c;
    ds.offsets[e] = o;
    off[e] = o;
    for (int m0 = 0; m0 < c; m0 += DEC_MT) ds.tiles[tb++] = make_int4(e, o + m0, min(DEC_MT, c - m0), 0);
    o += c;
  }
  const int total = __shfl(c_inc, 63, 64), routed = __shfl(t_inc, 63, 64);
  const int nsh = has_shared ? (T + DEC_MT - 1) / DEC_MT : 0;
  if (lane < nsh) ds.tiles[routed + lane] = make_int4(E, lane * DEC_MT, min(DEC_MT, T - lane * DEC_MT), 0);
  if (lane == 0) {
    ds.offsets[E] = total;
    *ds.n_tiles = routed + nsh;
  }
  __builtin_amdgcn_wave_barrier();
  // placement: rank of token t among the tokens of expert e
  for (int i = lane; i < T * k; i += 64) {
    const int t = i / k, e = s_idx[i];
    const int pos = off[e] + __popc(msk[e] & ((1u << t) - 1u));
    ds.perm[pos] = i;
    ds.inv[i] = pos;
    ds.ptok[pos] = t;
  }
}

template <int NV>
__global__ __launch_bounds__(1024) void k_select_small(const float *__restrict__ logits,
                                                       const float *__restrict__ sgl,
                                                       const uint16_t *__restrict__ x,
                                                       int32_t *__restrict__ topk_idx,
                                                       float *__restrict__ topk_w,
                                                       float *__restrict__ sgate,
                                                       uint16_t *__restrict__ xperm, int T, int E,
                                                       int k, int H, int has_shared, int has_gate,
                                                       DispatchOut ds, int fused) {
  __shared__ int s_idx[SMALL_MT * 32];
  __shared__ uint32_t s_msk[1024];
  __shared__ int s_off[1024];
  __shared__ uint64_t s_cand[SMALL_MT][64];
  __shared__ uint64_t s_sel[SMALL_MT][16];
  const int t = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (t < T) {
    const float *ar = logits + (size_t)t * E;
    uint32_t key[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int e = lane + 64 * i;
      const float v = ar[min(e, E - 1)];  // unconditional: loads issue together
      key[i] = e < E ? ordered_key(v) : 0u;
    }
    int seli;
    uint32_t selk;
    wave_topk_fast<NV>(key, E, k, lane, seli, selk, s_cand[t], s_sel[t]);
    const float selv = lane < k ? ar[seli] : 0.0f;
    const float vmax = __shfl(selv, 0, 64);
    const float p = lane < k ? expf(selv - vmax) : 0.0f;
    float sum = 0.0f;
    for (int j = 0; j < k; ++j) sum += __shfl(p, j, 64);
    if (lane < k) {
      topk_idx[(size_t)t * k + lane] = seli;
      topk_w[(size_t)t * k + lane] = p / sum;
      s_idx[t * k + lane] = seli;
    }
    if (lane == 0) sgate[t] = has_gate ? 1.0f / (1.0f + expf(-sgl[t])) : 1.0f;
    if (xperm) write_xperm(x + (size_t)t * H, xperm, nullptr, t, H, lane);
  }
  if (!fused) return;
  __syncthreads();
  if (t == 0) dispatch_wave(s_idx, T, k, E, has_shared, ds, s_msk, s_off, lane);
}

template <int NV, bool EXACT, bool COOP>
hipError_t launch_select_nv(int ch, unsigned grid, const float *approx, const float *sgl,
                            const float *wnorm,
                            const void *x, const void *rw, const float *bias, const void *gw,
                            int32_t *idx, float *w, float *sg, void *xperm, float *xsum, int T,
                            int E, int k, int H, int has_shared, const DispatchOut &ds, int fused,
                            unsigned long long *cmask, int32_t *ccount, hipStream_t s) {
#define SEL_ARGS                                                                            \
  approx, sgl, wnorm, (const uint16_t *)x, (const uint16_t *)rw, bias, (const uint16_t *)gw, idx, \
      w, sg, (uint16_t *)xperm, xsum, T, E, k, H, has_shared, ds, fused, cmask, ccount
  switch (ch) {
  case 1: k_select<NV, 1, EXACT, COOP><<<grid, 256, 0, s>>>(SEL_ARGS); break;
  case 2: k_select<NV, 2, EXACT, COOP><<<grid, 256, 0, s>>>(SEL_ARGS); break;
  case 4: k_select<NV, 4, EXACT, COOP><<<grid, 256, 0, s>>>(SEL_ARGS); break;
  default: k_select<NV, 8, EXACT, COOP><<<grid, 256, 0, s>>>(SEL_ARGS); break;
  }
#undef SEL_ARGS
  return hipGetLastError();
}

}  // namespace

bool router_supported(int H, int E) { return H % 128 == 0 && H <= 4096 && E <= 1024; }

template <bool EXACT>
hipError_t launch_select(const float *approx, const float *sgl, const float *wnorm,
                         const void *x, const void *rw, const float *bias, const void *gw,
                         int32_t *idx, float *w, float *sg, void *xperm, float *xsum, int T,
                         int H, int E, int k, int has_shared, const DispatchOut *fused,
                         hipStream_t s, unsigned long long *cmask = nullptr,
                         int32_t *ccount = nullptr) {
  const int ch = (H / 8 + 63) / 64;  // chunks per lane
  const int chp = ch <= 1 ? 1 : (ch <= 2 ? 2 : (ch <= 4 ? 4 : 8));
  const int nv = (E + 63) / 64;
  DispatchOut ds;
  memset(&ds, 0, sizeof ds);
  if (fused) ds = *fused;
  // one token per workgroup below the GEMM path (k_select, COOP)
  const bool coop = !EXACT && T < GEMM_MIN_T;
  const unsigned g = coop ? (unsigned)T : (T + SEL_WAVES - 1) / SEL_WAVES;
  const int fz = fused ? 1 : 0;
#define SEL_CALL(NVV)                                                                          \
  (coop ? launch_select_nv<NVV, EXACT, !EXACT>(chp, g, approx, sgl, wnorm, x, rw, bias, gw, idx, \
                                              w, sg, xperm, xsum, T, E, k, H, has_shared, ds, \
                                              fz, cmask, ccount, s)                           \
        : launch_select_nv<NVV, EXACT, false>(chp, g, approx, sgl, wnorm, x, rw, bias, gw, idx, \
                                              w, sg, xperm, xsum, T, E, k, H, has_shared, ds, \
                                              fz, cmask, ccount, s))
  if (nv <= 1) return SEL_CALL(1);
  if (nv <= 2) return SEL_CALL(2);
  if (nv <= 4) return SEL_CALL(4);
  if (nv <= 8) return SEL_CALL(8);
  return SEL_CALL(16);
#undef SEL_CALL
}

hipError_t launch_router_fast(const void *x, const void *rw, const float *bias, const void *gw,
                              float *approx, float *wnorm, int32_t *idx, float *w, float *sg,
                              void *xperm, float *xsum, int T, int H, int E, int k,
                              int has_shared, const DispatchOut *fused, hipStream_t s,
                              int32_t *ccount, unsigned long long *cmask) {
  if (T == 0) return hipSuccess;
  // ---- approximate logits + row norms ------------------------------------
  if (T >= GEMM_MIN_T) {
    // (and the chunk counts and masks zeroed: [ccount, cmask end), which
    // k_select fills for the dispatch)
    const size_t zb = cmask ? (size_t)((char *)(cmask + (size_t)((T + 63) / 64) * E) - (char *)ccount) : 0;
    hipError_t err = launch_router_gemm(x, rw, bias, approx, wnorm, T, H, E, (uint32_t *)ccount,
                                        (int)(zb / 4), s);
    if (err != hipSuccess) return err;
    return launch_select<false>(approx, nullptr, wnorm, x, rw, bias, gw, idx, w, sg, xperm,
                                xsum, T, H, E, k, has_shared, fused, s, cmask, ccount);
  }
  // one 16-token tile per workgroup: more workgroups share the token reads
  // (c3 T=64: 55 -> 44 us against 64-token tiles; the router rows are
  // re-read from L2)
  constexpr int MS = 1;
  const int mt = 16 * MS;
  // decode: one token tile, K split over up to 16 waves; prefill: 4 waves
  int NW = T <= 64 ? H / 128 : 4;
  if (NW > 16) NW = 16;
  while (NW > 1 && (H % (32 * NW))) --NW;
  const dim3 grid((E + 15) / 16, (T + mt - 1) / mt);
  const size_t lds = sizeof(float) * ((size_t)NW * MS * 256 + NW * 16);
  k_router_mfma<MS><<<grid, NW * 64, lds, s>>>((const uint16_t *)x, (const uint16_t *)rw, bias,
                                               approx, wnorm, fused ? fused->ticket : nullptr, T,
                                               H, E, NW);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  // ---- refine + select ------------------------------------------------------
  return launch_select<false>(approx, nullptr, wnorm, x, rw, bias, gw, idx, w, sg, xperm, xsum,
                              T, H, E, k, has_shared, fused, s);
}

hipError_t launch_router_exact(const void *x, const void *rw, const float *bias, const void *gw,
                               float *logits, float *sg_logit, int32_t *idx, float *w, float *sg,
                               void *xperm, int T, int H, int E, int k, int has_shared,
                               const DispatchOut *fused, hipStream_t s) {
  if (T == 0) return hipSuccess;
  hipError_t err = launch_router(x, rw, bias, gw, logits, sg_logit,
                                 fused ? fused->ticket : nullptr, T, H, E, s);
  if (err != hipSuccess) return err;
  if (T > SMALL_MT) return hipErrorInvalidValue;
  DispatchOut ds;
  memset(&ds, 0, sizeof ds);
  if (fused) ds = *fused;
  const int nv = (E + 63) / 64;
#define SMALL_CALL(NVV)                                                                      \
  k_select_small<NVV><<<1, 64 * T, 0, s>>>(logits, sg_logit, (const uint16_t *)x, idx, w, sg,  \
                                          (uint16_t *)xperm, T, E, k, H, has_shared,          \
                                          gw ? 1 : 0, ds, fused ? 1 : 0)
  if (nv <= 1) SMALL_CALL(1);
  else if (nv <= 2) SMALL_CALL(2);
  else if (nv <= 4) SMALL_CALL(4);
  else if (nv <= 8) SMALL_CALL(8);
  else SMALL_CALL(16);
#undef SMALL_CALL
  return hipGetLastError();
}
