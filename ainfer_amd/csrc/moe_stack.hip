// moe_stack.hip - the persistent decode-stack kernel: L decoder-block MLP
// halves (RMSNorm -> MoE layer -> residual add, ainfer_moe_block_forward) at
// T <= 4 tokens in one launch.
//
// The per-block path pays three kernel launches per block (routing, gate/up,
// down + combine), each with its ramp and drain, and a block's down weights
// are only requested once its gate/up launch has finished.  Here one grid of
// G resident workgroups (G from the occupancy query, so every workgroup runs
// at once) walks the L layers.  Per layer:
//
//  1. routing, by the first NRW = ceil(rows / 8) workgroups: wave w takes
//     router row 8 * wg + w for all T tokens.  Wave t < T first normalizes
//     token t's residual row (the block's RMSNorm) into LDS; the dot runs in
//     the canonical lane-strided order of the oracle.  Workgroup 0 also
//     writes the normalized rows in MFMA order for the gate/up items.  Each
//     routing workgroup then arrives on the layer's logits counter;
//  2. selection, in every workgroup (no handoff): once the counter is full,
//     one wave per token reads the token's E + 1 logits, takes the exact
//     top-k, the renormalised weights and the shared gate; the dispatch
//     (tiles of at most DEC_MT tokens) is built in LDS;
//  3. items, dealt round-robin over the workgroups: gate/up items, then down
//     items; a down item issues its weight loads, then waits for its tile's
//     gate/up flags;
//  4. combine units (token, row slab), dealt from workgroup 0 again: each
//     waits for the down flags of the token's k + 1 tiles, writes the new
//     residual rows and arrives on the layer's residual counter, which every
//     workgroup waits for before the next layer.
//
// Coherence.  The L2 of each XCD is not coherent with the others'.  Every
// buffer a layer writes (logits, normalized x, act, o, the residual rows)
// lives in a region of its own per layer, written with sc1 stores (through
// to the coherence point) and read only after the wait that follows its
// writes: no workgroup has read those addresses earlier in the kernel, and
// kernel boundaries invalidate the L2s, so the reads are ordinary cached
// loads, served by each XCD's L2 after its first miss (device-coherent reads
// of data every workgroup shares would all go to the same memory channel).
// Only the waits themselves read device-coherently: one counter word each
// for the two all-workgroup waits (a 64-bit (tag << 32 | arrivals) word whose
// first arrival of a layer resets it, so nothing is cleared between calls),
// and per-item flags (tag) for the item-to-item waits.  Tags come from a host
// counter (tag0 + layer), so none repeats between calls.  No wait names work
// that comes later in any workgroup's own sequence, so with all workgroups
// resident every wait ends; waits are bounded all the same (a timeout sets
// the workspace's error word, and the combines then write NaN).
//
// The items are the per-block path's own (expert_lds_item, same K split and
// templates) and the combine sums in the same order, so each layer's output
// is bit-identical to ainfer_moe_block_forward's.
#include <string.h>

#include <mutex>
#include <type_traits>

#include "moe_common.h"
#include "moe_decode_parts.h"
#include "moe_expert_item.h"
#include "moe_internal.h"
#include "moe_topk.h"

#ifdef AINFER_STACK_TRACE
// debug builds only: per (layer, workgroup) timestamps of the phases
// (s_memrealtime, 100 MHz), layers below 8, workgroups below 1024
__device__ unsigned long long g_strace[8][1024][12];
#define STRACE(L, I)                                                      \
  if (threadIdx.x == 0 && (L) < 8 && blockIdx.x < 1024)                  \
  g_strace[L][blockIdx.x][I] = __builtin_amdgcn_s_memrealtime()
extern "C" int ainfer_debug_stack_trace(void *host) {
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(g_strace), sizeof(g_strace)) == hipSuccess ? 0 : -1;
}
// finer stamps inside the phases (after the wave's memory work lands)
__device__ unsigned long long g_strace2[8][1024][8];
#define STRACE2(L, I)                                                     \
  do {                                                                    \
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");                      \
    if ((threadIdx.x & 63) == 0 && (L) < 8 && blockIdx.x < 1024)          \
      g_strace2[L][blockIdx.x][I] = __builtin_amdgcn_s_memrealtime();      \
  } while (0)
extern "C" int ainfer_debug_stack_trace2(void *host) {
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(g_strace2), sizeof(g_strace2)) == hipSuccess ? 0 : -1;
}
#else
#define STRACE(L, I)
#define STRACE2(L, I)
#endif

namespace {

constexpr int STK_NW = 8;  // waves per workgroup
constexpr int STK_T = DECODE_NORM_MAX_T;
constexpr int STK_NB = 8;  // 16-byte chunks per lane of a row: H <= 4096
constexpr int STK_NREL = 64;  // release lines per counter (waiters spread over them)

struct StackArgs {
  const StackLayer *layers;
  int L;
  const uint16_t *x0;  // the stack's input rows [T][H]
  uint16_t *out;       // the stack's output rows [T][H]
  int T, H, E, k, I, Is, has_shared;
  int norm_mode;
  float eps;
  uint64_t *cnt;       // [8] counters, 32 words apart: logits [0..3], residual [4..7]
  int32_t *rel;        // [2][STK_NREL] release lines, 32 words apart: logits, residual
  int32_t *fgu, *fdn;  // [cap][slabs] routed item flags
  int32_t *fsgu, *fsdn;  // [slabs] shared-expert item flags
  int32_t *fx;           // the normalized rows (MFMA order) are written
  uint8_t *pl;         // per-layer regions, `stride` bytes apart
  size_t stride, off_lg, off_xp, off_act, off_acts, off_o, off_res;
  int32_t *err;
  uint32_t tag0;
  int wk_gu, wr_gu, slabs_gu, wk_dn, wr_dn, slabs_dn, nrw;
  int spin;
};

// the pieces of layer l's region
struct LayerBufs {
  float *lg;        // [T][E + 1] logits (slot E: the shared gate)
  uint16_t *xp;     // [T][H] normalized x, MFMA order
  uint16_t *act;    // [T * k][I]
  uint16_t *act_s;  // [T][Is]
  uint16_t *o;      // [T * k + T][H]
  const uint16_t *x;  // the layer's input rows
  uint16_t *res;      // the layer's output rows
};
__device__ __forceinline__ LayerBufs layer_bufs(const StackArgs &a, int l) {
  LayerBufs b;
  uint8_t *p = a.pl + (size_t)l * a.stride;
  b.lg = (float *)(p + a.off_lg);
  b.xp = (uint16_t *)(p + a.off_xp);
  b.act = (uint16_t *)(p + a.off_act);
  b.act_s = (uint16_t *)(p + a.off_acts);
  b.o = (uint16_t *)(p + a.off_o);
  b.x = l == 0 ? a.x0 : (const uint16_t *)(p - a.stride + a.off_res);
  b.res = l == a.L - 1 ? a.out : (uint16_t *)(p + a.off_res);
  return b;
}

__device__ __forceinline__ void st_dev16(__amdgpu_buffer_rsrc_t r, uint32_t off, u32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, CPOL_SC1);
}

// One wave: every flag f[0..n) equal to tag (bounded; spin 0 gives up at once).
__device__ __forceinline__ bool wave_wait_flags(const int32_t *f, int n, uint32_t tag, int spin,
                                                int lane) {
  for (int it = 0;; ++it) {
    bool ok = true;
    for (int i = lane; i < n; i += 64) ok &= (uint32_t)ld_dev(f + i) >= tag;
    if (spin > 0 && __all(ok)) return true;
    if (it >= spin) return false;
    __builtin_amdgcn_s_sleep(4);
  }
}

// Workgroup-wide: wave 0 waits, a timeout sets the error word.
__device__ __forceinline__ void wg_wait_flags(const int32_t *f, int n, uint32_t tag,
                                              const StackArgs &a) {
  if (threadIdx.x < 64) {
    const bool ok = wave_wait_flags(f, n, tag, a.spin, threadIdx.x);
    if (!ok && threadIdx.x == 0) atomicOr(a.err, 1);
  }
  __syncthreads();
}

// Arrival on a (tag << 32 | count) counter by one wave.  Tags only grow (a
// host counter), so the max of (tag << 32) resets a word that holds an older
// tag to (tag, 0) and leaves one that holds this tag alone; every arrival does
// its own max before its add (one address: performed in order), so the count
// is exact and no compare-and-swap retries (one memory round trip each at
// every contender) are needed.  The n-th arrival writes the tag to the
// STK_NREL release lines, one per lane: waiters poll the line of their own
// workgroup, so a few hundred of them do not all read one line (a hot line's
// polls queue in front of the arrivals and stores on its memory channel).
// Every wait compares >= tag, so a waiter that sees a later layer's tag has
// not missed its own.
__device__ __forceinline__ void arrive(uint64_t *c, int32_t *rel, uint32_t tag, int n,
                                       int lane) {
  unsigned long long old = 0;
  if (lane == 0) {
    atomicMax((unsigned long long *)c, (unsigned long long)tag << 32);
    old = atomicAdd((unsigned long long *)c, 1ull);
  }
  old = __shfl(old, 0, 64);
  if (old == (((unsigned long long)tag << 32) | (unsigned)(n - 1)) && lane < STK_NREL)
    st_dev(rel + 32 * lane, (int32_t)tag);
}

// Workgroup-wide wait for a release line (>= tag); thread 0 polls.
__device__ __forceinline__ void wg_wait_rel(const int32_t *rel, uint32_t tag,
                                            const StackArgs &a) {
  if (threadIdx.x == 0) {
    const int32_t *line = rel + 32 * (blockIdx.x % STK_NREL);
    bool ok = false;
    for (int it = 0; it < a.spin; ++it) {
      if ((uint32_t)ld_dev(line) >= tag) {
        ok = true;
        break;
      }
      __builtin_amdgcn_s_sleep(4);
    }
    if (!ok) atomicOr(a.err, 1);
  }
  __syncthreads();
}

// inv of a row from its squares summed in any order by one wave (chunks held
// by the lanes, valid where ok[b]).  The rare sequential re-sum reads row xr.
template <int N>
__device__ __forceinline__ float wave_rms_inv(const u32x4 (&v)[N], const bool (&ok)[N],
                                              const uint16_t *xr, int H, float eps, int lane) {
  double p4[4] = {0.0, 0.0, 0.0, 0.0};
  u16x2_t ek = {0x7F80, 0x7F80};
#pragma unroll
  for (int b = 0; b < N; ++b)
    if (ok[b]) sumsq_chunk(v[b], p4, ek);
  const double tot = wave_sum_f64((p4[0] + p4[1]) + (p4[2] + p4[3]));
  const int emin = (int)wave_min_u32((uint32_t)ek_emin(ek));
  return rms_inv_finish(tot, emin, xr, H, eps, lane);
}

// Token t's row normalized by the block's RMSNorm into LDS (canonical order,
// bf16): xl[t * H + j].  One wave.
__device__ __forceinline__ void norm_row_to_lds(const StackArgs &a, const StackLayer &ly,
                                                const uint16_t *x, int t, uint16_t *xl,
                                                int lane, int l) {
  const int H = a.H, nch = H >> 3;
  const uint16_t *xr = x + (size_t)t * H;
  u32x4 xv[STK_NB];
  bool ok[STK_NB];
#pragma unroll
  for (int b = 0; b < STK_NB; ++b) {
    ok[b] = lane + 64 * b < nch;
    xv[b] = *(const u32x4 *)(xr + (size_t)min(lane + 64 * b, nch - 1) * 8);
  }
  if (t == 0) STRACE2(l, 0);
  const float inv = wave_rms_inv<STK_NB>(xv, ok, xr, H, a.eps, lane);
  if (t == 0) STRACE2(l, 1);
  NormIn n;
  n.w = (const uint16_t *)ly.norm_w;
  n.mode = a.norm_mode;
  n.eps = a.eps;
  n.on = 1;
#pragma unroll
  for (int b = 0; b < STK_NB; ++b) {
    if (!ok[b]) continue;
    const int c = lane + 64 * b;
    const u32x4 nv = n.w ? *(const u32x4 *)(n.w + (size_t)c * 8) : u32x4{0u, 0u, 0u, 0u};
    u32x4 xx = xv[b];
#pragma unroll
    for (int q = 0; q < 4; ++q) xx[q] = norm_pair(xx[q], nv[q], inv, n);
    *(u32x4 *)(xl + (size_t)t * H + c * 8) = xx;
  }
}

// Logits of router row r (E: the shared gate row) for the T tokens whose
// normalized rows are in LDS, in k_route_decode's fma order (lane l: chunks
// l, l + 64, ... in order, then the xor butterfly).  wv: the row's chunks.
__device__ __forceinline__ void router_row_load(const StackArgs &a, const StackLayer &ly, int r,
                                                u32x4 (&wv)[STK_NB], int lane) {
  const int H = a.H, nch = H >> 3;
  const uint16_t *wr = r < a.E ? (const uint16_t *)ly.w.router_w + (size_t)r * H
                               : (const uint16_t *)ly.w.shared_gate_w;
#pragma unroll
  for (int b = 0; b < STK_NB; ++b)
    wv[b] = *(const u32x4 *)(wr + (size_t)min(lane + 64 * b, nch - 1) * 8);
}
__device__ __forceinline__ void router_row_logits(const StackArgs &a, const StackLayer &ly,
                                                  const u32x4 (&wv)[STK_NB], const uint16_t *xl,
                                                  int r, float *lg, int lane) {
  const int H = a.H, E = a.E, nch = H >> 3;
  for (int t = 0; t < a.T; ++t) {
    float acc = 0.0f;
#pragma unroll
    for (int b = 0; b < STK_NB; ++b) {
      const bool ok = lane + 64 * b < nch;
      const u32x4 x = *(const u32x4 *)(xl + (size_t)t * H + min(lane + 64 * b, nch - 1) * 8);
      float s = acc;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        s = __builtin_fmaf(__uint_as_float(x[q] << 16), __uint_as_float(wv[b][q] << 16), s);
        s = __builtin_fmaf(__uint_as_float(x[q] & 0xFFFF0000u),
                           __uint_as_float(wv[b][q] & 0xFFFF0000u), s);
      }
      acc = ok ? s : acc;
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) acc = acc + __shfl_xor(acc, m, 64);
    if (lane == 0) {
      const float v = r < E && ly.w.router_bias ? acc + ly.w.router_bias[r] : acc;
      st_dev((uint32_t *)lg + (size_t)t * (E + 1) + r, __float_as_uint(v));
    }
  }
}

// Token t's normalized row (LDS) written in MFMA order (write_xperm's layout)
// with sc1 stores.  One wave.
__device__ __forceinline__ void xperm_row(const StackArgs &a, const uint16_t *xl, uint16_t *xp,
                                          int t, int lane) {
  const int H = a.H, nblk = H >> 5;
  const __amdgpu_buffer_rsrc_t xo = make_rsrc(xp + (size_t)t * H, H * 2);
  for (int b = lane; b < nblk; b += 64) {
    uint32_t in[16];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const u32x4 v = *(const u32x4 *)(xl + (size_t)t * H + b * 32 + j * 8);
#pragma unroll
      for (int q = 0; q < 4; ++q) in[4 * j + q] = v[q];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t o4[4];
#pragma unroll
      for (int e2 = 0; e2 < 4; ++e2) {
        const int ka = 8 * e2 + j, kb = ka + 4;
        const uint32_t lo = (in[ka >> 1] >> (16 * (ka & 1))) & 0xFFFFu;
        const uint32_t hi = (in[kb >> 1] >> (16 * (kb & 1))) & 0xFFFFu;
        o4[e2] = lo | (hi << 16);
      }
      st_dev16(xo, (uint32_t)(b * 32 + j * 8) * 2, u32x4{o4[0], o4[1], o4[2], o4[3]});
    }
  }
}

// Arguments of layer l's items: mode 0 = gate/up (+ SiLU), 1 = down.
__device__ __forceinline__ ExpertArgs item_args(const StackArgs &a, const StackLayer &ly,
                                                const LayerBufs &b, const int32_t *ptok,
                                                int mode) {
  ExpertArgs e;
  memset(&e, 0, sizeof e);
  e.ptok = ptok;
  e.T = a.T;
  e.k = a.k;
  e.E = a.E;
  e.H = a.H;
  e.I = a.I;
  e.Is = a.Is;
  if (mode == 0) {
    e.w0 = ly.w.w_gate;
    e.w1 = ly.w.w_up;
    e.s0 = (const uint16_t *)ly.w.s_gate;
    e.s1 = (const uint16_t *)ly.w.s_up;
    e.ws0 = ly.w.ws_gate;
    e.ws1 = ly.w.ws_up;
    e.ss0 = (const uint16_t *)ly.w.ss_gate;
    e.ss1 = (const uint16_t *)ly.w.ss_up;
    e.a_routed = b.xp;
    e.a_shared = b.xp;
    e.act = b.act;
    e.act_s = b.act_s;
    e.WK = a.wk_gu;
    e.WR = a.wr_gu;
    e.n_slabs = a.slabs_gu;
  } else {
    e.w0 = ly.w.w_down;
    e.s0 = (const uint16_t *)ly.w.s_down;
    e.ws0 = ly.w.ws_down;
    e.ss0 = (const uint16_t *)ly.w.ss_down;
    e.a_routed = b.act;
    e.a_shared = b.act_s;
    e.o = b.o;
    e.WK = a.wk_dn;
    e.WR = a.wr_dn;
    e.n_slabs = a.slabs_dn;
  }
  return e;
}

#ifndef STK_WAVES_PER_EU
#define STK_WAVES_PER_EU 4  // register budget: 2 workgroups of 8 waves per CU (<= 128 VGPRs);
                            // 6 (3 per CU, 80 VGPRs) spills more: c4 T=1 layer 59.5 -> 50.6 us
#endif
template <int SD, int NV, int KBW_DN>
__global__ __launch_bounds__(STK_NW * 64, STK_WAVES_PER_EU) void k_decode_stack(StackArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  __shared__ uint64_t s_cand[STK_T][68];
  __shared__ uint64_t s_sel[STK_T][16];
  __shared__ int s_idx[STK_T * 32];
  __shared__ float s_w[STK_T * 32], s_sg[STK_T];
  __shared__ int s_perm[STK_T * 32], s_inv[STK_T * 32], s_ptok[STK_T * 32], s_p2t[STK_T * 32];
  __shared__ int4 s_tiles[STK_T * 32 + STK_T];
  __shared__ int s_ntiles;
  const int G = gridDim.x, wg = blockIdx.x;
  const int T = a.T, H = a.H, E = a.E, k = a.k;
  DispatchOut ds;
  memset(&ds, 0, sizeof ds);
  ds.perm = s_perm;
  ds.inv = s_inv;
  ds.ptok = s_ptok;
  ds.tiles = s_tiles;
  ds.n_tiles = &s_ntiles;
  ds.mt = DEC_MT;
  const int rows_dn = 16 * DEC_RG_DOWN * a.wr_dn;
  const int sg = a.slabs_gu, sd = a.slabs_dn;
  u32x4 wv[STK_NB];  // routing workgroups: this layer's router row, in flight

  for (int l = 0; l < a.L; ++l) {
    const uint32_t tag = a.tag0 + (uint32_t)l;
    int wave = tid_opaque() >> 6, lane = tid_opaque() & 63;
    // the layer's table entry is read where it is used (scalar loads), so no
    // copy of it stays live across the phases
    const StackLayer &ly = a.layers[l];
    const LayerBufs lb = layer_bufs(a, l);
    uint64_t *c_lg = a.cnt + 32 * (l & 3), *c_res = a.cnt + 32 * (4 + (l & 3));
    int32_t *rel_lg = a.rel, *rel_res = a.rel + 32 * STK_NREL;
    STRACE(l, 0);
    // ---- 0. the previous layer's residual rows are all written ----------
    if (l > 0) wg_wait_rel(rel_res, tag - 1u, a);
    STRACE(l, 1);
    // ---- 1. routing: workgroups [0, NRW), one router row per wave; the
    // row's loads were issued before the residual wait ---------------------
    const bool has_gate = ly.w.shared_gate_w != nullptr;
    const int nrows = E + (has_gate ? 1 : 0);
    const int r_mine = wg * STK_NW + wave;
    if (wg < a.nrw) {
      uint16_t *xl = (uint16_t *)lds;  // the items' LDS, idle now
      if (l == 0 && r_mine < nrows) router_row_load(a, ly, r_mine, wv, lane);
      if (wave < T) norm_row_to_lds(a, ly, lb.x, wave, xl, lane, l);
      if (wave == 0) STRACE2(l, 2);
      __syncthreads();
      STRACE(l, 2);
      if (wg == 0 && wave < T) {
        xperm_row(a, xl, lb.xp, wave, lane);
        wait_stores();
      }
      if (wg == 0) {
        __syncthreads();
        if (threadIdx.x == 0) st_dev(a.fx, (int32_t)tag);
      }
      if (r_mine < nrows) router_row_logits(a, ly, wv, xl, r_mine, lb.lg, lane);
      wait_stores();
      if (wave == 0) STRACE2(l, 3);
      __syncthreads();
      if (threadIdx.x < 64) arrive(c_lg, rel_lg, tag, a.nrw, threadIdx.x);
    }
    STRACE(l, 3);
    // ---- 1b. the shared expert's gate/up items: independent of the
    // routing, on workgroups after the routing ones, as soon as x is
    // normalized (its down items lead the main list's down section) --------
    const int nsh = a.has_shared ? 1 : 0;  // one shared tile: T <= DEC_MT
    const int4 tsh = make_int4(E, 0, T, 0);
    if (nsh) {
      for (int q = (wg - a.nrw + G) % G; q < sg; q += G) {
        lane = tid_opaque() & 63;
        __syncthreads();
        const ExpertArgs gu = item_args(a, ly, lb, s_ptok, 0);
        const int32_t *fx = a.fx;
        expert_lds_item<SD, 4, DEC_RG_GATE_UP, DEC_MT, 0, true, false>(
            gu, tsh, q, lds, [&]() { wg_wait_flags(fx, 1, tag, a); });
        if (threadIdx.x < 64) {
          wait_stores();
          if (lane == 0) st_dev(a.fsgu + q, (int32_t)tag);
        }
      }
    }
    // ---- 2. selection and dispatch, in every workgroup -------------------
    wg_wait_rel(rel_lg, tag, a);
    STRACE(l, 4);
    wave = tid_opaque() >> 6;
    lane = tid_opaque() & 63;
    if (wave < T) {
      const int t = wave;
      const float *lgt = lb.lg + (size_t)t * (E + 1);
      uint32_t key[NV];
#pragma unroll
      for (int i = 0; i < NV; ++i)
        key[i] = lane + 64 * i < E ? ordered_key(lgt[min(lane + 64 * i, E - 1)]) : 0u;
      const float sgl = has_gate ? lgt[E] : 0.0f;
      int seli;
      uint32_t selk;
      wave_topk_fast<NV>(key, E, k, lane, seli, selk, s_cand[t], s_sel[t]);
      const float selv = lane < k ? key_to_float(selk) : 0.0f;
      const float vmax = __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(selv)));
      const float p = lane < k ? expf(selv - vmax) : 0.0f;
      float sum = 0.0f;  // in pick order, as the oracle
      for (int j = 0; j < k; ++j) sum += __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(p), j));
      if (lane < k) {
        s_idx[t * k + lane] = seli;
        s_w[t * k + lane] = p / sum;
      }
      if (lane == 0) s_sg[t] = has_gate ? 1.0f / (1.0f + expf(-sgl)) : 1.0f;
      if (T == 1) {
        // one token: the tiles are its k picks in expert order (position =
        // rank among the picks), then the shared tile -- dispatch_decode's
        // output for T = 1
        int rank = 0;
        for (int j = 0; j < k; ++j)
          rank += __builtin_amdgcn_readlane(seli, j) < seli ? 1 : 0;
        if (lane < k) {
          s_tiles[rank] = make_int4(seli, rank, 1, 0);
          s_ptok[rank] = 0;
          s_inv[lane] = rank;
        }
        if (lane == 0) {
          if (a.has_shared) s_tiles[k] = make_int4(E, 0, 1, 0);
          s_ntiles = k + nsh;
        }
      }
    }
    __syncthreads();
    if (T > 1) {
      dispatch_decode<STK_NW>(s_idx, T, k, E, a.has_shared, ds);
      __syncthreads();
    }
    const int n_tiles = s_ntiles;
    for (int ti = threadIdx.x; ti < n_tiles - nsh; ti += STK_NW * 64) {
      const int4 td = s_tiles[ti];
      for (int m = 0; m < td.z; ++m) s_p2t[td.y + m] = ti;
    }
    __syncthreads();
    STRACE(l, 5);
    // ---- 3. items: gate/up, then down, round-robin over workgroups; then
    // 4. the combine units, dealt from workgroup 0 again: their count does
    // not depend on the routing, so each runs exactly once even if
    // workgroups disagreed on the tiles (a timed-out wait) ------------------
    // items: the routed gate/up items, the shared expert's down items, the
    // routed down items.  Dealt round-robin from workgroup nrw + sg on, so the
    // routing workgroups and those that ran the shared gate/up items (both
    // start this phase late) come last and take fewer items.
    const int n_rt = n_tiles - nsh;  // the routed tiles
    const int n_gu = n_rt * sg, n_sdn = nsh * sd, n_dn = n_rt * sd, n_cb = T * sd;
    const int n_items = n_gu + n_sdn + n_dn;
    const int wr = (wg - (a.nrw + nsh * sg) % G + G) % G;  // this workgroup's turn
    const int my_items = n_items > wr ? (n_items - wr + G - 1) / G : 0;
    const int my_cb = n_cb > wg ? (n_cb - wg + G - 1) / G : 0;
    for (int i = 0; i < my_items + my_cb; ++i) {
      STRACE(l, 6 + (i < 5 ? i : 5));
      // q: item index, or n_items + combine unit index
      const int q = i < my_items ? wr + i * G : n_items + wg + (i - my_items) * G;
      lane = tid_opaque() & 63;
      __syncthreads();  // the previous item's LDS (read by its wave 0) is free
      if (q < n_gu) {
        const int tile = q / sg, slab = q % sg;
        const ExpertArgs gu = item_args(a, ly, lb, s_ptok, 0);
        expert_lds_item<SD, 4, DEC_RG_GATE_UP, DEC_MT, 0, true, false>(gu, s_tiles[tile], slab,
                                                                        lds);
        if (threadIdx.x < 64) {
          wait_stores();
          if (lane == 0) st_dev(a.fgu + tile * sg + slab, (int32_t)tag);
        }
      } else if (q < n_gu + n_sdn) {
        const int slab = q - n_gu;
        const int32_t *fg = a.fsgu;
        const ExpertArgs dn = item_args(a, ly, lb, s_ptok, 1);
        expert_lds_item<SD, KBW_DN, DEC_RG_DOWN, DEC_MT, 1, true, false>(
            dn, tsh, slab, lds, [&]() { wg_wait_flags(fg, sg, tag, a); });
        if (threadIdx.x < 64) {
          wait_stores();
          if (lane == 0) st_dev(a.fsdn + slab, (int32_t)tag);
        }
      } else if (q < n_items) {
        const int tile = (q - n_gu - n_sdn) / sd, slab = (q - n_gu - n_sdn) % sd;
        const int32_t *fg = a.fgu + tile * sg;
        const ExpertArgs dn = item_args(a, ly, lb, s_ptok, 1);
        expert_lds_item<SD, KBW_DN, DEC_RG_DOWN, DEC_MT, 1, true, false>(
            dn, s_tiles[tile], slab, lds, [&]() { wg_wait_flags(fg, sg, tag, a); });
        if (threadIdx.x < 64) {
          wait_stores();
          if (lane == 0) st_dev(a.fdn + tile * sd + slab, (int32_t)tag);
        }
      } else {
        // ---- combine of (token t, row slab), slot order (k_combine's) ----
        const int c = q - n_items, t = c / sd, slab = c % sd;
        bool okw = true;
        if (threadIdx.x < 64) {
          // the down items of the token's k routed tiles and its shared tile
          int wt = -1;
          if (lane < k) wt = s_p2t[s_inv[t * k + lane]];
          const int32_t *fw = lane < k ? a.fdn + wt * sd + slab
                                       : (lane == k && a.has_shared ? a.fsdn + slab : nullptr);
          for (int it = 0;; ++it) {
            const bool ok = fw == nullptr || (uint32_t)ld_dev(fw) >= tag;
            if (a.spin > 0 && __all(ok)) break;
            if (it >= a.spin) {
              okw = false;
              break;
            }
            __builtin_amdgcn_s_sleep(4);
          }
          if (!okw && lane == 0) atomicOr(a.err, 1);
          STRACE2(l, 4);
          const int r0 = slab * rows_dn;
          const size_t Tk = (size_t)T * k;
          // this unit's own wait, or any earlier one on the workspace, ran out
          const bool bad = !okw || ld_dev(a.err) != 0;
          const __amdgpu_buffer_rsrc_t rr = make_rsrc(lb.res, (uint32_t)(T * H * 2));
          constexpr int CB = 4;  // slots whose loads are issued together
          for (int hr = lane; hr < rows_dn; hr += 64) {
            const int h = min(r0 + hr, H - 1);
            float acc = 0.0f;
            for (int j0 = 0; j0 < k; j0 += CB) {
              uint16_t ov[CB];
              float wj[CB];
#pragma unroll
              for (int j = 0; j < CB; ++j) {
                const int jj = min(j0 + j, k - 1);
                const int pos = s_inv[t * k + jj];
                wj[j] = s_w[t * k + jj];
                ov[j] = lb.o[(size_t)pos * H + h];
              }
#pragma unroll
              for (int j = 0; j < CB; ++j)
                if (j0 + j < k) acc = __builtin_fmaf(wj[j], bf16_to_f32(ov[j]), acc);
            }
            if (a.has_shared)
              acc = __builtin_fmaf(s_sg[t], bf16_to_f32(lb.o[(Tk + t) * H + h]), acc);
            acc += bf16_to_f32(lb.x[(size_t)t * H + h]);
            if (r0 + hr < H)
              st_dev_u16(rr, (uint32_t)(((size_t)t * H + h) * 2),
                         bad ? (uint16_t)0x7FC0u : f32_to_bf16(acc));
          }
          wait_stores();
          STRACE2(l, 5);
        }
        __syncthreads();
        if (threadIdx.x < 64) arrive(c_res, rel_res, tag, n_cb, threadIdx.x);
        if (threadIdx.x < 64) STRACE2(l, 6);
      }
    }
    __syncthreads();
    // the next layer's router row: its loads fly over the residual wait
    if (wg < a.nrw && l + 1 < a.L) {
      const StackLayer &ln = a.layers[l + 1];
      const int rn = wg * STK_NW + (tid_opaque() >> 6);
      if (rn < a.E + (ln.w.shared_gate_w ? 1 : 0)) router_row_load(a, ln, rn, wv, tid_opaque() & 63);
    }
    STRACE(l, 11);
  }
}

uint32_t g_stack_tag = 0;
std::mutex g_stack_mu;

}  // namespace

bool stack_geometry(const ainfer_moe_shape &s, int T, StackGeom *g) {
  if (s.precision != AINFER_PRECISION_W4A16) return false;  // the W4A16 items only
  DecodeGeom dg;
  if (!decode_geometry(s, &dg)) return false;
  int kbw, wk, wr;
  if (!expert_geometry(0, s.hidden, s.inter, s.shared_inter, 4, &kbw, &wk, &wr) || kbw != 4)
    return false;
  g->wk_gu = wk;
  // down: the per-block path's K split at this token count (T <= 2: the
  // fused expert kernel's KBW 2, else the stand-alone kernels' down_kbw)
  g->kbw_dn = T <= FUSED_EXPERTS_MAX_T ? 2 : down_kbw_of(s);
  if (!expert_geometry(1, s.hidden, s.inter, s.shared_inter, g->kbw_dn, &kbw, &wk, &wr) ||
      kbw != g->kbw_dn)
    return false;
  g->wk_dn = wk;
  if (g->wk_gu > STK_NW || g->wk_dn > STK_NW || STK_NW % g->wk_gu || STK_NW % g->wk_dn)
    return false;
  g->wr_gu = STK_NW / g->wk_gu;
  g->wr_dn = STK_NW / g->wk_dn;
  const int Ngu = s.inter > s.shared_inter ? s.inter : s.shared_inter;
  g->slabs_gu = (Ngu + 16 * DEC_RG_GATE_UP * g->wr_gu - 1) / (16 * DEC_RG_GATE_UP * g->wr_gu);
  g->slabs_dn = (s.hidden + 16 * DEC_RG_DOWN * g->wr_dn - 1) / (16 * DEC_RG_DOWN * g->wr_dn);
  const size_t l_gu = (size_t)STK_NW * item_lds_per_wave(DEC_MT, 4, DEC_RG_GATE_UP, 0);
  const size_t l_dn = (size_t)STK_NW * item_lds_per_wave(DEC_MT, g->kbw_dn, DEC_RG_DOWN, 1);
  g->lds = l_gu > l_dn ? l_gu : l_dn;
  const size_t l_x = (size_t)STK_T * s.hidden * 2;  // the routing's normalized rows
  if (g->lds < l_x) g->lds = l_x;
  g->nw = STK_NW;
  return g->lds <= 64 * 1024 && s.n_experts <= 1024 && s.top_k <= 32;
}

int stack_flag_words(const ainfer_moe_shape &s, int cap) {
  StackGeom g;
  int slabs_gu = 0, slabs_dn = 0;
  for (int T = 1; T <= STK_T; ++T)
    if (stack_geometry(s, T, &g)) {
      slabs_gu = slabs_gu > g.slabs_gu ? slabs_gu : g.slabs_gu;
      slabs_dn = slabs_dn > g.slabs_dn ? slabs_dn : g.slabs_dn;
    }
  // counters (8 x 256 B), release lines, the routed item flags, the shared
  // ones, fx
  return 8 * 64 + 2 * STK_NREL * 32 + cap * (slabs_gu + slabs_dn) + slabs_gu + slabs_dn + 64;
}

static size_t al256(size_t v) { return (v + 255) & ~(size_t)255; }

size_t stack_layer_bytes(const ainfer_moe_shape &s, int T, size_t *offs) {
  const size_t H = s.hidden, E = s.n_experts, k = s.top_k, I = s.inter,
               Is = s.shared_inter > 0 ? s.shared_inter : 1;
  size_t off = 0, o[6];
  o[0] = off; off += al256((size_t)T * (E + 1) * 4);   // logits
  o[1] = off; off += al256((size_t)T * H * 2);         // normalized x (MFMA order)
  o[2] = off; off += al256((size_t)T * k * I * 2);     // act
  o[3] = off; off += al256((size_t)T * Is * 2);        // act_s
  o[4] = off; off += al256((size_t)(T * k + T) * H * 2);  // o
  o[5] = off; off += al256((size_t)T * H * 2);         // the layer's output rows
  if (offs)
    for (int i = 0; i < 6; ++i) offs[i] = o[i];
  return off;
}

hipError_t launch_decode_stack(int scale_dtype, const ainfer_moe_shape &s, const StackGeom &g,
                               const StackLayer *layers, int L, const void *x0, void *out, int T,
                               int norm_mode, float eps, const StackWs &w, hipStream_t st) {
  if (L <= 0 || T <= 0) return hipSuccess;
  if (T > STK_T) return hipErrorInvalidValue;
  StackArgs a;
  memset(&a, 0, sizeof a);
  a.layers = layers;
  a.L = L;
  a.x0 = (const uint16_t *)x0;
  a.out = (uint16_t *)out;
  a.T = T;
  a.H = s.hidden;
  a.E = s.n_experts;
  a.k = s.top_k;
  a.I = s.inter;
  a.Is = s.shared_inter;
  a.has_shared = s.shared_inter > 0;
  a.norm_mode = norm_mode;
  a.eps = eps;
  a.cnt = (uint64_t *)w.flags;
  a.rel = w.flags + 8 * 64;
  a.fgu = a.rel + 2 * STK_NREL * 32;
  a.fdn = a.fgu + w.cap * g.slabs_gu;
  a.fsgu = a.fdn + w.cap * g.slabs_dn;
  a.fsdn = a.fsgu + g.slabs_gu;
  a.fx = a.fsdn + g.slabs_dn;
  size_t offs[6];
  a.stride = stack_layer_bytes(s, T, offs);
  a.pl = w.layers;
  a.off_lg = offs[0];
  a.off_xp = offs[1];
  a.off_act = offs[2];
  a.off_acts = offs[3];
  a.off_o = offs[4];
  a.off_res = offs[5];
  a.err = w.err;
  a.wk_gu = g.wk_gu;
  a.wr_gu = g.wr_gu;
  a.slabs_gu = g.slabs_gu;
  a.wk_dn = g.wk_dn;
  a.wr_dn = g.wr_dn;
  a.slabs_dn = g.slabs_dn;
  a.nrw = (s.n_experts + 1 + STK_NW - 1) / STK_NW;
  a.spin = g_spin_max;
  {
    // tags tag0 .. tag0 + L - 1, never 0 and never those of the previous
    // call (counters and flags start at 0 after ainfer_moe_workspace_init)
    std::lock_guard<std::mutex> lock(g_stack_mu);
    if (g_stack_tag + (uint32_t)L + 2u < g_stack_tag) g_stack_tag = 0;
    a.tag0 = g_stack_tag + 2u;
    g_stack_tag += (uint32_t)L + 1u;
  }
  int dev = 0, cus = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return e;
  const int nv = (a.E + 63) / 64;
  auto go = [&](auto sd_c, auto nv_c, auto kb_c) -> hipError_t {
    constexpr int SDc = decltype(sd_c)::value, NVc = decltype(nv_c)::value,
                  KBc = decltype(kb_c)::value;
    auto kern = k_decode_stack<SDc, NVc, KBc>;
    int per_cu = 0;
    hipError_t e2 = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, STK_NW * 64, g.lds);
    if (e2 != hipSuccess) return e2;
    if (per_cu < 1) return hipErrorInvalidConfiguration;
    if (per_cu > 3) per_cu = 3;
    if (cus * per_cu < a.nrw) return hipErrorInvalidConfiguration;
    kern<<<cus * per_cu, STK_NW * 64, g.lds, st>>>(a);
    return hipGetLastError();
  };
  auto by_kb = [&](auto sd_c, auto nv_c) -> hipError_t {
    if (g.kbw_dn == 4) return go(sd_c, nv_c, std::integral_constant<int, 4>());
    return go(sd_c, nv_c, std::integral_constant<int, 2>());
  };
  auto by_nv = [&](auto sd_c) -> hipError_t {
    if (nv <= 1) return by_kb(sd_c, std::integral_constant<int, 1>());
    if (nv <= 2) return by_kb(sd_c, std::integral_constant<int, 2>());
    if (nv <= 4) return by_kb(sd_c, std::integral_constant<int, 4>());
    if (nv <= 8) return by_kb(sd_c, std::integral_constant<int, 8>());
    return by_kb(sd_c, std::integral_constant<int, 16>());
  };
  if (scale_dtype == AINFER_SCALE_FP16) return by_nv(std::integral_constant<int, AINFER_SCALE_FP16>());
  return by_nv(std::integral_constant<int, AINFER_SCALE_BF16>());
}
