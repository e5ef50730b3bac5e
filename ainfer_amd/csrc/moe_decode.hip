// moe_decode.hip - the decode routing kernel (T <= 16 tokens) and the fused
// expert kernel (T <= 2).
//
// Measured on MI355X: a dependent kernel launch costs about 2.5 us, a flag
// handed from one workgroup to another through device memory about 0.8 us,
// same-address device atomics serialise at about 11 ns each, and an
// agent-scope release or acquire fence (a whole-L2 write-back or
// invalidate) about 20 ns, serialised.  So at T = 2 the layer is two kernels
// whose stages meet through counters that few workgroups touch, with data
// handed over by sc1 stores and loads instead of fences (moe_common.h):
//
//  k_route_decode   workgroups [0, NR): canonical router logits, one
//                   (one row x 1 or 2 tokens) unit per wave, each stored
//                   with an sc1 store as ~bits into a key slot of the sync
//                   region (never 0: ~bits == 0 only for one NaN pattern no
//                   bf16 product or sum yields); workgroup NR (one wave per
//                   token) polls its token's slots
//                   until none is 0, clears them, takes the exact top-k, the
//                   weights and the shared gate, and builds the dispatch
//                   (tiles of at most DEC_MT tokens) from LDS.  A slot that is
//                   its own ready flag saves the store wait, barrier and
//                   counter round trip of an arrival.  Workgroup NR + 1
//                   writes x in MFMA order meanwhile.
//  k_experts_decode one workgroup per item: first every gate/up + SiLU item
//                   (tile-major, slab-minor), one arrival each on
//                   gu_done[tile]; then every down item, which requests its
//                   weights, waits for gu_done[tile] == gate/up slabs, reads
//                   the tile's act rows, writes its o rows, and counts one
//                   arrival per (token, row slab).  The (k+1)-th arrival of a
//                   (token, slab) sums the token's k + 1 rows of that slab in
//                   slot order (the combine).  At T = 1 the gate/up items
//                   run first in a launch of their own (k_expert_lds) and
//                   this kernel holds only the down items, which then wait
//                   for nothing.
//
// A wait only ever names work of lower workgroup index, and workgroups are
// dispatched in index order, so every awaited workgroup is already running.
// Waits are bounded (SPIN_MAX polls); one that runs out sets the error word
// of the sync region and carries on.  The error word is sticky: while it is
// set, every combine (this kernel's and k_combine) writes NaN outputs, so a
// call whose handoff failed, and every later call on that workspace until
// ainfer_moe_workspace_init clears it, returns visibly bad rows rather than
// silently wrong ones (a late arrival can leave a counter non-zero, which
// would let a later call's waits pass early).
//
// Every counter is reset by its last user (the logit slots by the selection
// workgroup, gu_done/dn_done by a tile's last down item, a (token, slab)
// counter by its last arrival), so the sync region is zero again when a call
// ends.  It must be zero before the first call (ainfer_moe_workspace_init).
//
// Debug builds with -DAINFER_DECODE_TRACE record per-workgroup timestamps.
#include <string.h>

#include <type_traits>

#include "moe_common.h"
#include "moe_expert_item.h"
#include "moe_internal.h"
#include "moe_topk.h"
#include "moe_decode_parts.h"

#ifdef AINFER_DECODE_TRACE
// debug builds only: per-workgroup timestamps (s_memrealtime, 100 MHz)
__device__ unsigned long long g_dtrace[2][1 << 15][5];
#define DTRACE_AT(K, X, I) \
  if (threadIdx.x == 0 && (X) < (1 << 15)) g_dtrace[K][X][I] = __builtin_amdgcn_s_memrealtime()
#define DTRACE(K, I) DTRACE_AT(K, blockIdx.x, I)
extern "C" int ainfer_debug_trace(void *host) {
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(g_dtrace), sizeof(g_dtrace)) == hipSuccess ? 0 : -1;
}
extern "C" int ainfer_debug_land(void *host) {
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(g_dland), sizeof(g_dland)) == hipSuccess ? 0 : -1;
}
#else
#define DTRACE(K, I)
#define DTRACE_AT(K, X, I)
#endif

namespace {

constexpr int RD_WAVES = 16;  // waves per k_route_decode workgroup
// Router units: one router row x TT tokens per wave (TT = 1 up to
// RD_TT1_MAX tokens, else 2: more, shorter units shorten the routing at few
// tokens; measured at T = 1, 4, 16 against 2 rows x 4 tokens: -2.9, -3.4,
// -0.5 us per layer).  At TT = 1 the workgroups have RD_W1 waves and a lane
// issues the loads of its whole row at once (c3 T=1: -1 us).
constexpr int RD_R = 1;       // router rows per wave
constexpr int RD_TT1_MAX = 4;
constexpr int RD_NB = 2;      // 8-element chunks per lane whose loads are issued together
#ifndef RD_W1
#define RD_W1 4    // waves per workgroup at T <= RD_TT1_MAX (the rows spread over more CUs)
#endif
#ifndef RD_NB1
#define RD_NB1 8   // chunks in flight at T <= RD_TT1_MAX: a whole row up to H = 4096
#endif
// RD_TT1_MAX < T <= RD_W2: two tokens per wave in workgroups of RD_W2 waves
// with RD_NB2 chunks in flight, so the 2048 units of c4 T=8 spread over all
// CUs instead of half of them (16-wave workgroups, which T > RD_W2 needs for
// its one selection wave per token).  c4 T=8 routing stage 13.8 -> 12.2 us
// per block; one token per wave in 8-wave workgroups: 12.4 us.
#ifndef RD_W2
#define RD_W2 8
#endif
#ifndef RD_NB2
#define RD_NB2 4
#endif
#ifndef RD_MID_TT
#define RD_MID_TT 2
#endif
static_assert(RD_W1 >= RD_TT1_MAX, "the selection runs one wave per token");
static_assert(DECODE_NORM_MAX_T <= RD_TT1_MAX, "the folded RMSNorm exists in the TT = 1 form only");
constexpr int SPIN_MAX = 1 << 20;
#ifndef DEC_WAVES_PER_SIMD
#define DEC_WAVES_PER_SIMD 6  // register budget of the expert kernel (<= 80 VGPRs)
#endif
#ifndef DEC_NW_MIN
#define DEC_NW_MIN 4  // waves per expert workgroup (at least)
#endif
#ifndef DEC_RG_GU
#define DEC_RG_GU 1  // 16-row groups per wave, gate/up items (16 x 2 rows x H)
#endif
#ifndef DEC_RG_DN
#define DEC_RG_DN 2  // 16-row groups per wave, down items
#endif

struct RouteDecodeArgs {
  const uint16_t *x, *rw, *gw;
  const float *bias;
  float *logits, *sgl;  // [T][E], [T]
  int32_t *idx;
  float *w, *sg;
  uint16_t *xperm;
  int8_t *w8q;      // optional: W4A8 codes and group scales of the (normalized) x
  float *w8sq;
  DispatchOut ds;
  int32_t *sync;
  uint32_t *slots;  // [DECODE_MAX_T][E + 1] ~bits of the logits (sync region)
  NormIn norm;      // on: x is the residual stream, normalized here (RMSNorm)
  int T, H, E, k, has_shared, NR;
  int spin;         // polls before a wait gives up (0: at once)
};

// W waves per workgroup (T <= W: the selection runs one wave per token), NB
// chunks of 8 per lane whose loads are issued together
// NORM: x is the residual stream and the block's RMSNorm is applied here
// (T <= RD_TT1_MAX only: at two tokens per wave the extra registers cost
// more than the saved launch)
template <int NV, int RD_TT, int W, int NB, bool NORM>
__global__ __launch_bounds__(W * 64) void k_route_decode(RouteDecodeArgs a) {
  __shared__ uint64_t s_cand[W][68];
  __shared__ uint64_t s_sel[W][16];
  __shared__ int s_idx[W * 32];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int T = a.T, H = a.H, E = a.E, k = a.k;
  DTRACE(0, 0);
  if ((int)blockIdx.x < a.NR) {
    // ---- canonical logits of RD_R rows x RD_TT tokens per wave: lane l
    // sums 8-element chunks l, l+64, ... with fma in order, then the xor
    // butterfly (the oracle's mo_router_dot) ---------------------------------
    const int nrows = E + (a.gw ? 1 : 0);
    const int ngroups = (nrows + RD_R - 1) / RD_R;
    const int u = blockIdx.x * W + wave;
    const int rbase = (u % ngroups) * RD_R, t0 = (u / ngroups) * RD_TT;
    if (t0 < T) {
      const uint16_t *wr[RD_R];
#pragma unroll
      for (int i = 0; i < RD_R; ++i) {
        const int r = min(rbase + i, nrows - 1);
        wr[i] = r < E ? a.rw + (size_t)r * H : a.gw;
      }
      const int nch = H >> 3;
      // RMSNorm folded in: each token's scale from the x chunks the loop
      // below loads (the whole row: one pass, H <= 64 * NB * 8), then x
      // normalized per chunk
      static_assert(!NORM || 64 * NB * 8 >= 4096, "the folded RMSNorm needs the whole row");
      float inv[RD_TT];
#pragma unroll
      for (int j = 0; j < RD_TT; ++j) inv[j] = 1.0f;
      float acc[RD_R][RD_TT];
#pragma unroll
      for (int i = 0; i < RD_R; ++i)
#pragma unroll
        for (int j = 0; j < RD_TT; ++j) acc[i][j] = 0.0f;
      // NB chunks' loads in flight at once; the sums still run over
      // chunks l, l + 64, ... in order
      for (int cb = lane; cb < nch; cb += 64 * NB) {
        u32x4 wv[NB][RD_R], xv[NB][RD_TT], nv[NB];
        // x and the norm weight first: loads complete in issue order, so the
        // RMSNorm (which needs only them) runs while the router row, a cold
        // read from HBM, is still in flight
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          const int c = min(cb + 64 * b, nch - 1);
#pragma unroll
          for (int j = 0; j < RD_TT; ++j)
            xv[b][j] = *(const u32x4 *)(a.x + (size_t)min(t0 + j, T - 1) * H + (size_t)c * 8);
          nv[b] = NORM && a.norm.w ? *(const u32x4 *)(a.norm.w + (size_t)c * 8)
                                   : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          const int c = min(cb + 64 * b, nch - 1);
#pragma unroll
          for (int i = 0; i < RD_R; ++i) wv[b][i] = *(const u32x4 *)(wr[i] + (size_t)c * 8);
        }
        if constexpr (NORM) {
          // sum of squares in any order (rms_mean_f's tests hold for every
          // order), four independent fp64 chains per lane
#pragma unroll
          for (int j = 0; j < RD_TT; ++j) {
            double p4[4] = {0.0, 0.0, 0.0, 0.0};
            u16x2_t ek = {0x7F80, 0x7F80};
#pragma unroll
            for (int b = 0; b < NB; ++b)
              if (cb + 64 * b < nch) sumsq_chunk(xv[b][j], p4, ek);
            int emin = ek_emin(ek);
            // wave reductions on the DPP path (no LDS round trips on this
            // critical path); one value in every lane
            const double tot = wave_sum_f64((p4[0] + p4[1]) + (p4[2] + p4[3]));
            emin = (int)wave_min_u32((uint32_t)emin);
            inv[j] = rms_inv_finish(tot, emin, a.x + (size_t)min(t0 + j, T - 1) * H, H,
                                    a.norm.eps, lane);
          }
#pragma unroll
          for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int j = 0; j < RD_TT; ++j)
#pragma unroll
              for (int q = 0; q < 4; ++q) xv[b][j][q] = norm_pair(xv[b][j][q], nv[b][q], inv[j], a.norm);
          DTRACE(0, 2);
        }
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          // past the row end: computed on a clamped chunk and discarded, so
          // no load depends on a branch
          const bool in = cb + 64 * b < nch;
#pragma unroll
          for (int i = 0; i < RD_R; ++i)
#pragma unroll
            for (int j = 0; j < RD_TT; ++j) {
              float s = acc[i][j];
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                s = __builtin_fmaf(__uint_as_float(xv[b][j][q] << 16), __uint_as_float(wv[b][i][q] << 16), s);
                s = __builtin_fmaf(__uint_as_float(xv[b][j][q] & 0xFFFF0000u),
                                   __uint_as_float(wv[b][i][q] & 0xFFFF0000u), s);
              }
              acc[i][j] = in ? s : acc[i][j];
            }
        }
      }
#pragma unroll
      for (int m = 32; m >= 1; m >>= 1)
#pragma unroll
        for (int i = 0; i < RD_R; ++i)
#pragma unroll
          for (int j = 0; j < RD_TT; ++j) acc[i][j] = acc[i][j] + __shfl_xor(acc[i][j], m, 64);
      DTRACE(0, 3);
      if (lane == 0) {
#pragma unroll
        for (int i = 0; i < RD_R; ++i)
#pragma unroll
          for (int j = 0; j < RD_TT; ++j) {
            const int r = rbase + i, t = t0 + j;
            if (r >= nrows || t >= T) continue;
            const float v = r < E && a.bias ? acc[i][j] + a.bias[r] : acc[i][j];
            st_dev(a.slots + (size_t)t * (E + 1) + r, ~__float_as_uint(v));
          }
      }
    }
    DTRACE(0, 1);
    return;
  }
  const int t = wave;
  if ((int)blockIdx.x > a.NR) {
    // ---- workgroup NR + 1: the MFMA-order copy of x, one wave per token.
    // It does not depend on the routing; a workgroup of its own keeps it off
    // the selection's path (the selection polls as soon as it starts).
    if (t < T && a.xperm) {
      const float inv = NORM ? row_rms_inv(a.x + (size_t)t * H, H, a.norm.eps, lane) : 1.0f;
      write_xperm(a.x + (size_t)t * H, a.xperm, nullptr, t, H, lane, NORM ? &a.norm : nullptr, inv,
                  a.w8q, a.w8sq);
    }
    return;
  }
  // ---- the selection workgroup (NR): one wave per token (T <= W) ----------
  uint32_t raw[NV], graw = 0u;
  if (t < T) {
    uint32_t *sl = a.slots + (size_t)t * (E + 1);
    // poll the token's slots until every one is written (bounded)
    for (int it = 0;; ++it) {
#pragma unroll
      for (int i = 0; i < NV; ++i) raw[i] = ld_dev(sl + min(lane + 64 * i, E - 1));
      graw = ld_dev(sl + E);  // the shared gate's slot (stays 0 without one)
      uint32_t nz = graw | (a.gw ? 0u : 1u);
#pragma unroll
      for (int i = 0; i < NV; ++i) nz = min(nz, raw[i]);
      if (a.spin > 0 && __all(nz != 0u)) break;
      if (it >= a.spin) {
        if (lane == 0) atomicOr(a.sync + SY_ERR, 1);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    DTRACE(0, 4);
    uint32_t key[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) key[i] = lane + 64 * i < E ? ordered_key(__uint_as_float(~raw[i])) : 0u;
    const float sgl = __uint_as_float(~graw);
    int seli;
    uint32_t selk;
    wave_topk_fast<NV>(key, E, k, lane, seli, selk, s_cand[wave], s_sel[wave]);
    DTRACE(0, 1);
    const float selv = lane < k ? key_to_float(selk) : 0.0f;
    const float vmax = __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(selv)));
    const float p = lane < k ? expf(selv - vmax) : 0.0f;
    float sum = 0.0f;  // in pick order, as the oracle
    for (int j = 0; j < k; ++j) sum += __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(p), j));
    if (lane < k) {
      a.idx[(size_t)t * k + lane] = seli;
      a.w[(size_t)t * k + lane] = p / sum;
      s_idx[t * k + lane] = seli;
    }
    if (lane == 0) a.sg[t] = a.gw ? 1.0f / (1.0f + expf(-sgl)) : 1.0f;
  }
  DTRACE(0, 2);
  __syncthreads();
  if (a.ds.tiles) dispatch_decode<W>(s_idx, T, k, E, a.has_shared, a.ds);
  DTRACE(0, 3);
  // off the critical path: the logits output, and the slots cleared for
  // the next call
  if (t < T) {
    uint32_t *sl = a.slots + (size_t)t * (E + 1);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int e = lane + 64 * i;
      if (e < E) {
        st_dev(sl + e, 0u);
        a.logits[(size_t)t * E + e] = __uint_as_float(~raw[i]);
      }
    }
    if (a.gw && lane == 0) {
      st_dev(sl + E, 0u);
      a.sgl[t] = __uint_as_float(~graw);
    }
  }
}

struct ExpertsDecodeArgs {
  ExpertArgs gu, dn;  // WK, WR, n_slabs set (WK * WR waves in both)
  const float *w, *sg;
  const int32_t *inv;
  const uint16_t *resid;
  uint16_t *y;
  int32_t *sync;
  int max_tiles, cap;  // grid tiles; capacity of the per-tile counter arrays
  int spin;            // polls before a wait gives up (0: at once)
};

// One item per workgroup.  A down item only ever waits for gate/up items of
// lower index, which the dispatcher has started, so the waits end.
// SPLIT: the gate/up items ran in an earlier launch (k_expert_lds): this
// launch holds only the down items, which need no wait and read act with
// plain (cacheable) loads.
template <int SD, int KBW_GU, int RG_GU, int KBW_DN, int RG_DN, bool SPLIT>
__global__ __launch_bounds__(1024, DEC_WAVES_PER_SIMD) void k_experts_decode(ExpertsDecodeArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  // one counter per 256-byte line: same-line atomics and polls serialise
  int32_t *gu_done = a.sync + SY_TILES, *dn_done = gu_done + a.cap * SY_STRIDE,
          *cnt = dn_done + a.cap * SY_STRIDE;
  const int lane = threadIdx.x & 63;
  const int sg = a.gu.n_slabs, sd = a.dn.n_slabs;
  const int n_gu = a.max_tiles * sg;
  {
    const int item = blockIdx.x + (SPLIT ? n_gu : 0);
    // ---- item -> (kind, tile, slab): all gate/up items (tile-major,
    // slab-minor), then all down items ---------------------------------------
    const int is_gu = item < n_gu;
    const int r = is_gu ? item : item - n_gu, ns = is_gu ? sg : sd;
    const int tile = r / ns, slab = r % ns;
    int n_tiles;
    const int4 tt = sload_tile(is_gu ? a.gu.tiles : a.dn.tiles, a.gu.n_tiles, tile, n_tiles);
    if (tile >= n_tiles) return;
    DTRACE_AT(1, item, 0);
#ifdef AINFER_DECODE_TRACE
    if (threadIdx.x == 0) g_dtrace[1][item][4] = is_gu;
#endif
    // one item per workgroup, and no barrier before its loads: each wave
    // issues its weight loads as soon as it is launched (the waves of a
    // workgroup start up to about 1.5 us apart at the launch's start)
    if (!SPLIT && is_gu) {
      // x (MFMA order) comes from the routing kernel: plain, cacheable loads
      expert_lds_item<SD, KBW_GU, RG_GU, DEC_MT, 0, true, false>(a.gu, tt, slab, lds);
      if (threadIdx.x >= 64) return;
      // wave 0: its act stores, then the arrival
      DTRACE_AT(1, item, 2);
      wait_stores();
      if (lane == 0) atomicAdd(&gu_done[tile * SY_STRIDE], 1);
      DTRACE_AT(1, item, 3);
      return;
    }
    const int4 td = tt;
    // the down weights are requested before the wait for the tile's act rows
    const int32_t *gdone = &gu_done[tile * SY_STRIDE];
    int32_t *err = a.sync + SY_ERR;
    expert_lds_item<SD, KBW_DN, RG_DN, DEC_MT, 1, true, !SPLIT>(a.dn, td, slab, lds, [=]() {
      if (!SPLIT) block_wait_geq(gdone, sg, err, a.spin);
      DTRACE_AT(1, item, 1);
    });
    if (threadIdx.x >= 64) return;
    DTRACE_AT(1, item, 2);
    // ---- wave 0: publish o; count this tile's down items and each token's
    // arrivals on this row slab --------------------------------------------
    wait_stores();
    if (!SPLIT && lane == 0 && atomicAdd(&dn_done[tile * SY_STRIDE], 1) == sd - 1) {
      gu_done[tile * SY_STRIDE] = 0;  // all of the tile's down items have passed their wait
      dn_done[tile * SY_STRIDE] = 0;
    }
    const bool shared = td.x == a.dn.E;
    const int mcnt = td.z;
    const int has_shared = a.dn.Is > 0;
    const int k = a.dn.k, H = a.dn.H;
    int tok = -1;
    if (lane < mcnt) {
      const int pos = td.y + lane;
      const int tt = shared ? pos : a.dn.ptok[pos];
      int32_t *c = &cnt[(tt * sd + slab) * SY_STRIDE];
      if (atomicAdd(c, 1) == k + has_shared - 1) {
        *c = 0;
        tok = tt;
      }
    }
    DTRACE_AT(1, item, 3);
    if (__ballot(tok >= 0) == 0ull) return;
    // ---- combine of the completed (token, slab) pairs: slot order, as
    // k_combine -------------------------------------------------------------
    const __amdgpu_buffer_rsrc_t orr = make_rsrc(a.dn.o, 0x7FFFFFFFu);
    const int rows = 16 * RG_DN * a.dn.WR, r0 = slab * rows;
    const size_t Tk = (size_t)a.dn.T * k;
    // a wait of this or an earlier call on the workspace ran out (this
    // workgroup's own timeout is already visible here): NaN outputs
    const bool bad = __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
    constexpr int CB = 4;  // slots whose loads are issued together
    for (int i = 0; i < mcnt; ++i) {
      const int t = __builtin_amdgcn_readfirstlane(__shfl(tok, i, 64));
      if (t < 0) continue;
      for (int hr = lane; hr < rows; hr += 64) {
        const int h = min(r0 + hr, H - 1);
        float acc = 0.0f;
        for (int j0 = 0; j0 < k; j0 += CB) {
          uint16_t ov[CB];
          float wj[CB];
#pragma unroll
          for (int j = 0; j < CB; ++j) {
            const int jj = min(j0 + j, k - 1);
            const int pos = a.inv[(size_t)t * k + jj];
            wj[j] = a.w[(size_t)t * k + jj];
            ov[j] = ld_dev_u16(orr, (uint32_t)(((size_t)pos * H + h) * 2));
          }
#pragma unroll
          for (int j = 0; j < CB; ++j)
            if (j0 + j < k) acc = __builtin_fmaf(wj[j], bf16_to_f32(ov[j]), acc);
        }
        if (has_shared)
          acc = __builtin_fmaf(a.sg[t],
                               bf16_to_f32(ld_dev_u16(orr, (uint32_t)(((Tk + t) * H + h) * 2))), acc);
        if (a.resid) acc += bf16_to_f32(a.resid[(size_t)t * H + h]);
        if (r0 + hr < H) a.y[(size_t)t * H + h] = bad ? (uint16_t)0x7FC0u : f32_to_bf16(acc);
      }
    }
  }
}

}  // namespace

int g_spin_max = SPIN_MAX;

int decode_geometry(const ainfer_moe_shape &s, DecodeGeom *g) {
  int kbw, wk, wr;
  if (!expert_geometry(0, s.hidden, s.inter, s.shared_inter, 4, &kbw, &wk, &wr) || kbw != 4)
    return 0;
  g->wk_gu = wk;
  if (!expert_geometry(1, s.hidden, s.inter, s.shared_inter, 2, &kbw, &wk, &wr) || kbw != 2)
    return 0;
  g->wk_dn = wk;
  g->nw = g->wk_gu > g->wk_dn ? g->wk_gu : g->wk_dn;
  if (g->nw < DEC_NW_MIN) g->nw = DEC_NW_MIN;
  if (g->nw % g->wk_gu || g->nw % g->wk_dn || g->nw > 16) return 0;
  g->wr_gu = g->nw / g->wk_gu;
  g->wr_dn = g->nw / g->wk_dn;
  const int Ngu = s.inter > s.shared_inter ? s.inter : s.shared_inter;
  g->slabs_gu = (Ngu + 16 * DEC_RG_GU * g->wr_gu - 1) / (16 * DEC_RG_GU * g->wr_gu);
  g->slabs_dn = (s.hidden + 16 * DEC_RG_DN * g->wr_dn - 1) / (16 * DEC_RG_DN * g->wr_dn);
  // A staging only: the K-split partials reuse it (expert_lds_item, COH)
  const size_t lds_gu = (size_t)g->nw * item_lds_per_wave(DEC_MT, 4, DEC_RG_GU, 0);
  const size_t lds_dn = (size_t)g->nw * item_lds_per_wave(DEC_MT, 2, DEC_RG_DN, 1);
  g->lds = lds_gu > lds_dn ? lds_gu : lds_dn;
  if (g->lds > 64 * 1024) return 0;
  return 1;
}

hipError_t launch_route_decode(const void *x, const void *rw, const float *bias, const void *gw,
                               float *logits, float *sgl, int32_t *idx, float *w, float *sg,
                               void *xperm, int T, int H, int E, int k, int has_shared,
                               const DispatchOut *ds, int32_t *sync, uint32_t *slots,
                               const NormIn *norm, hipStream_t s, int8_t *w8q, float *w8sq) {
  if (T <= 0) return hipSuccess;
  if (T > DECODE_MAX_T || T > RD_WAVES || E > 1024) return hipErrorInvalidValue;
  RouteDecodeArgs a;
  memset(&a, 0, sizeof a);
  a.x = (const uint16_t *)x;
  a.rw = (const uint16_t *)rw;
  a.gw = (const uint16_t *)gw;
  a.bias = bias;
  a.logits = logits;
  a.sgl = sgl;
  a.idx = idx;
  a.w = w;
  a.sg = sg;
  a.xperm = (uint16_t *)xperm;
  a.w8q = w8q;
  a.w8sq = w8sq;
  if (w8q && !xperm) return hipErrorInvalidValue;  // the codes come with the MFMA-order copy
  if (ds) a.ds = *ds;
  a.sync = sync;
  a.slots = slots;
  if (norm) a.norm = *norm;
  if (a.norm.on && T > RD_TT1_MAX) return hipErrorInvalidValue;  // see k_route_decode
  a.T = T;
  a.H = H;
  a.E = E;
  a.k = k;
  a.has_shared = has_shared;
  a.spin = g_spin_max;
  const int nrows = E + (gw ? 1 : 0);
  const bool mid = T > RD_TT1_MAX && T <= RD_W2;
  const int tt = T <= RD_TT1_MAX ? 1 : mid ? RD_MID_TT : 2;
  const int units = (nrows + RD_R - 1) / RD_R * ((T + tt - 1) / tt);
  const int wg = T <= RD_TT1_MAX ? RD_W1 : mid ? RD_W2 : RD_WAVES;
  a.NR = (units + wg - 1) / wg;
  const unsigned grid = a.NR + 2;  // router units, the selection, the x copy
  const int nv = (E + 63) / 64;
  auto go = [&](auto nv_c) {
    constexpr int NVc = decltype(nv_c)::value;
    if (T <= RD_TT1_MAX && a.norm.on)
      k_route_decode<NVc, 1, RD_W1, RD_NB1, true><<<grid, RD_W1 * 64, 0, s>>>(a);
    else if (T <= RD_TT1_MAX)
      k_route_decode<NVc, 1, RD_W1, RD_NB1, false><<<grid, RD_W1 * 64, 0, s>>>(a);
    else if (mid)
      k_route_decode<NVc, RD_MID_TT, RD_W2, RD_MID_TT == 1 ? RD_NB1 : RD_NB2, false>
          <<<grid, RD_W2 * 64, 0, s>>>(a);
    else
      k_route_decode<NVc, 2, RD_WAVES, RD_NB, false><<<grid, RD_WAVES * 64, 0, s>>>(a);
  };
  if (nv <= 1) go(std::integral_constant<int, 1>());
  else if (nv <= 2) go(std::integral_constant<int, 2>());
  else if (nv <= 4) go(std::integral_constant<int, 4>());
  else if (nv <= 8) go(std::integral_constant<int, 8>());
  else go(std::integral_constant<int, 16>());
  return hipGetLastError();
}

hipError_t launch_experts_decode(int scale_dtype, const DecodeGeom &g, ExpertArgs gu,
                                 ExpertArgs dn, const float *w, const float *sg,
                                 const int32_t *inv, const void *resid, void *y,
                                 int32_t *sync, int max_tiles, int cap, bool split,
                                 hipStream_t s) {
  if (max_tiles <= 0) return hipSuccess;
  if (max_tiles > cap) return hipErrorInvalidValue;
  ExpertsDecodeArgs a;
  memset(&a, 0, sizeof a);
  gu.WK = g.wk_gu;
  gu.WR = g.wr_gu;
  gu.n_slabs = g.slabs_gu;
  dn.WK = g.wk_dn;
  dn.WR = g.wr_dn;
  dn.n_slabs = g.slabs_dn;
  a.gu = gu;
  a.dn = dn;
  a.w = w;
  a.sg = sg;
  a.inv = inv;
  a.resid = (const uint16_t *)resid;
  a.y = (uint16_t *)y;
  a.sync = sync;
  a.max_tiles = max_tiles;
  a.cap = cap;
  a.spin = g_spin_max;
  const long grid = (long)max_tiles * (g.slabs_gu + g.slabs_dn);
  if (grid > 0x7FFFFFFF) return hipErrorInvalidValue;
  const int threads = g.nw * 64;
  if (split) {
    // the down items with the combine; the caller launched gate/up (the
    // same items, k_expert_lds) just before
    const long gd = (long)max_tiles * g.slabs_dn;
    if (scale_dtype == AINFER_SCALE_FP16)
      k_experts_decode<AINFER_SCALE_FP16, 4, DEC_RG_GU, 2, DEC_RG_DN, true><<<(unsigned)gd, threads, g.lds, s>>>(a);
    else
      k_experts_decode<AINFER_SCALE_BF16, 4, DEC_RG_GU, 2, DEC_RG_DN, true><<<(unsigned)gd, threads, g.lds, s>>>(a);
    return hipGetLastError();
  }
  if (scale_dtype == AINFER_SCALE_FP16)
    k_experts_decode<AINFER_SCALE_FP16, 4, DEC_RG_GU, 2, DEC_RG_DN, false><<<(unsigned)grid, threads, g.lds, s>>>(a);
  else
    k_experts_decode<AINFER_SCALE_BF16, 4, DEC_RG_GU, 2, DEC_RG_DN, false><<<(unsigned)grid, threads, g.lds, s>>>(a);
  return hipGetLastError();
}

__global__ void k_zero_i32(int32_t *p, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0;
}


hipError_t launch_zero_i32(int32_t *p, int n, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  k_zero_i32<<<(n + 255) / 256 < 1024 ? (n + 255) / 256 : 1024, 256, 0, s>>>(p, n);
  return hipGetLastError();
}
