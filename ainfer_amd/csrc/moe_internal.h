// moe_internal.h - host-side launchers shared between the kernel files and
// the C-ABI implementation (moe_api.hip).  Not part of the public ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/ainfer_moe.h"

// Arguments of the grouped expert kernels (one launch covers the routed
// experts and the shared expert, whose tiles carry expert id E).
struct ExpertArgs {
  const uint8_t *w0, *w1;     // routed: gate, up (MODE 0) or down (MODE 1)
  const uint16_t *s0, *s1;    // their scales
  const uint8_t *ws0, *ws1;   // shared expert tensors
  const uint16_t *ss0, *ss1;
  const uint16_t *a_routed;   // MODE 0: x in MFMA order [T][H]; MODE 1: act [Tk][I]
  const uint16_t *a_shared;   // MODE 0: same x; MODE 1: act_s [T][Is]
  uint16_t *act;              // MODE 0 out: [Tk][I] bf16, MFMA order
  uint16_t *act_s;            // MODE 0 out: [T][Is]
  uint16_t *o;                // MODE 1 out: [Tk + T][H] bf16
  const int32_t *ptok;        // token of each dispatch position
  const int4 *tiles;          // (expert, first position, rows, 0)
  const int32_t *n_tiles;
  int T, k, E, H, I, Is;
  int WK, WR, n_slabs;        // set by the launcher
};

// Arguments of the prefill GEMM (moe_gemm.hip).
struct GemmArgs {
  const uint8_t *w0, *w1;
  const uint16_t *s0, *s1;
  const uint8_t *ws0, *ws1;
  const uint16_t *ss0, *ss1;
  const uint16_t *a_routed;   // MODE 0: x in MFMA order [T][H]; MODE 1: act [Tk][I]
  const uint16_t *a_shared;   // MODE 1: act_s [T][Is]
  uint16_t *act, *act_s;      // MODE 0 out
  uint16_t *o;                // MODE 1 out: [Tk + T][H] bf16
  const float *xsum;          // [T][H/128] group sums of x
  float *asum, *asum_s;       // [Tk][I/32], [T][Is/32] (max) partial sums of act
  const int32_t *ptok;
  const int4 *tiles;
  const int32_t *n_tiles;
  int T, k, E, H, I, Is;
  int n_nblk, aslots;         // set by the launcher
};
// Prefill router: approximate logits (+ bias) and router row norms, tiled bf16 MFMA GEMM.
// zbuf: zwords 32-bit words zeroed by the kernel (the dispatch counts and
// masks the following k_select fills), or null
hipError_t launch_router_gemm(const void *x, const void *rw, const float *bias, float *approx,
                              float *wnorm, int T, int H, int E, uint32_t *zbuf, int zwords,
                              hipStream_t s);
hipError_t launch_expert_gemm(int mode, int scale_dtype, GemmArgs a, int max_tiles,
                              hipStream_t s);
// token-tile height of the prefill GEMM and the T above which it is used
constexpr int GEMM_MT = 128;
// experts with at most this many tokens leave the prefill GEMM (0: none)
#ifndef GEMM_SMALL_MAX
#define GEMM_SMALL_MAX 32
#endif
#ifndef GEMM_WN
#define GEMM_WN 4       // row waves per GEMM block (2 x GEMM_WN waves)
#endif
constexpr int GEMM_MIN_T = 256;

// Outputs of the dispatch stage.  tiles: (expert, first position, rows,
// first row within the expert); shared-expert tiles carry expert id E and a
// token base.  ptok[pos] = token of dispatch position pos.
// the combine arrival counters, zeroed by the dispatch.  ticket is the
// last-block counter of the fused top-k + dispatch launch.
struct DispatchOut {
  int32_t *counts, *offsets, *perm, *inv, *ptok;
  int4 *tiles;
  int32_t *n_tiles;
  int32_t *ticket;
  // experts with 1..small_max tokens get SMALL_MT-token tiles in tiles2
  // instead of tiles (small_max 0: no split)
  int4 *tiles2;
  int32_t *n_tiles2;
  int small_max;
  int mt;  // tokens per tile of dispatch_small_block
};

hipError_t launch_fill(int kind, uint64_t seed, float std_, size_t n, void *out,
                       hipStream_t s);
hipError_t launch_rmsnorm(const void *x, const void *w, int mode, float eps, void *y,
                          int T, int H, hipStream_t s);
// ticket (may be NULL) is zeroed for the fused top-k + dispatch launch
hipError_t launch_router(const void *x, const void *rw, const float *bias, const void *gw,
                         float *logits, float *sg_logit, int32_t *ticket, int T, int H, int E,
                         hipStream_t s);
// Router: approximate MFMA logits -> exact candidate refine -> top-k,
// weights, shared gate, MFMA-order copy of x.  fused != NULL (T <= 64 only):
// the last block also runs the dispatch.  approx [T][E] and wnorm [E] are
// scratch.
bool router_supported(int H, int E);
// xsum (may be NULL): [T][H/128] group sums of x for the prefill GEMM.
hipError_t launch_router_fast(const void *x, const void *rw, const float *bias, const void *gw,
                              float *approx, float *wnorm, int32_t *idx, float *w, float *sg,
                              void *xperm, float *xsum, int T, int H, int E, int k,
                              int has_shared, const DispatchOut *fused, hipStream_t s,
                              int32_t *ccount = nullptr, unsigned long long *cmask = nullptr);
// Small T: canonical logits of all experts on VALU (k_router_logits), then the
// same selection without the refine.  logits [T][E], sg_logit [T] out.
hipError_t launch_router_exact(const void *x, const void *rw, const float *bias, const void *gw,
                               float *logits, float *sg_logit, int32_t *idx, float *w, float *sg,
                               void *xperm, int T, int H, int E, int k, int has_shared,
                               const DispatchOut *fused, hipStream_t s);
// below this many tokens the router computes every logit in the canonical order
constexpr int EXACT_ROUTER_MAX_T = 16;
// cmask non-null: the per-(64-token chunk, expert) token masks (and, in
// chunk_counts, the counts) the router's k_select already built
// (T >= GEMM_MIN_T), so no counting launch
hipError_t launch_dispatch(const int32_t *idx, int T, int k, int E, int mt, int has_shared,
                           int32_t *chunk_counts, int32_t *rank, const DispatchOut &ds,
                           hipStream_t s, const unsigned long long *cmask = nullptr);
// x in MFMA order (+ its per-128 group sums when xsum is non-null)
hipError_t launch_xperm(const void *x, void *xperm, float *xsum, int T, int H, hipStream_t s);
// expert output rows from dispatch-position order to slot order (H % 8 == 0)
hipError_t launch_gather_rows(const void *src, const int32_t *inv, void *dst, int T, int k,
                              int H, int has_shared, hipStream_t s);
// inv null: o's routed rows are in slot order (row t * k + j)
hipError_t launch_combine(const uint16_t *o, const int32_t *inv, const float *w, const float *sg,
                          int has_shared, const void *resid, void *y, int T, int k, int H,
                          const int32_t *err, hipStream_t s);
// The same combine (resid non-null, H % 8 == 0, H <= 4096, 16-byte aligned
// rows) followed by the next block's RMSNorm of each written row:
// h[t] = RMSNorm(y[t]) with `next` (weight, mode, eps), bit-identical to
// launch_rmsnorm on y.  One 256-thread block per token.
hipError_t launch_combine_norm(const uint16_t *o, const int32_t *inv, const float *w,
                               const float *sg, int has_shared, const void *resid, void *y,
                               int T, int k, int H, const int32_t *err, const NormIn &next,
                               void *h, hipStream_t s);
// polls a bounded device wait makes before it gives up (sets the workspace's
// error word); ainfer_moe_debug_spin_limit changes it for tests
extern int g_spin_max;
// false when the shape has no wave geometry (more than 8 waves along K)
bool expert_geometry(int mode, int H, int I, int Is, int pref_kbw, int *KBW, int *WK,
                     int *WR);
// mode 0: gate/up + SiLU-mul; mode 1: down.  max_tiles bounds
// the tile list.
// pref_kbw: preferred 128-wide k-groups per wave (1, 2 or 4).
#ifndef RG_GATE_UP
#define RG_GATE_UP 1
#endif
#ifndef RG_DOWN
#define RG_DOWN 2
#endif
// the same for the decode tiles (T > FUSED_EXPERTS_MAX_T), and the down
// items' preferred k-groups per wave
#ifndef DEC_RG_GATE_UP
#define DEC_RG_GATE_UP 1
#endif
#ifndef DEC_RG_DOWN
#define DEC_RG_DOWN 2
#endif
#ifndef DEC_KBW_DOWN
#define DEC_KBW_DOWN 2
#endif
// rg: 16-row groups per wave (1, 2 or 4) sharing one load of the token rows;
// mt: tokens per tile the dispatch produced (DEC_MT: A staged in LDS, or SMALL_MT)
// The next decode gate/up launch of launch_expert_stream (the DEC_MT items)
// goes through hipExtLaunchKernel with these start/stop events (one shot).
void set_expert_launch_events(hipEvent_t start, hipEvent_t stop);
hipError_t launch_expert_stream(int mode, int scale_dtype, ExpertArgs a, int max_tiles,
                                int pref_kbw, int rg, int mt, hipStream_t s);

// tile height of the small-M expert kernels
constexpr int SMALL_MT = 16;
// LDS bytes per wave of a decode expert item (moe_expert_item.h): its A
// rows (MT x KBW * 256 B), its scales (KBW >= 2: one dword DMA per 256 B),
// and its K-split partials where they do not fit the A rows.
__host__ __device__ constexpr int item_scale_lds(int kbw, int rg, int mode) {
  return kbw >= 2 ? ((mode == 0 ? 2 : 1) * rg * 16 * kbw * 2 + 255) / 256 * 256 : 0;
}
__host__ __device__ constexpr int item_lds_per_wave(int mt, int kbw, int rg, int mode) {
  return mt * kbw * 256 + item_scale_lds(kbw, rg, mode) +
         (mt * kbw * 256 >= (mode == 0 ? 2 : 1) * rg * 1024 ? 0 : (mode == 0 ? 2 : 1) * rg * 1024);
}
constexpr int DEC_MT = 4;  // tile rows of the decode dispatch (T <= EXACT_ROUTER_MAX_T)
// largest T routed by the fused top-k + dispatch launch
constexpr int FUSED_DISPATCH_MAX_T = 64;


// ---- decode layer in two launches (moe_decode.hip), T <= DECODE_MAX_T ----
constexpr int DECODE_MAX_T = EXACT_ROUTER_MAX_T;
// ainfer_moe_block_forward folds the RMSNorm into the decode routing kernel
// up to this many tokens (its one-token-per-wave form)
constexpr int DECODE_NORM_MAX_T = 4;
// up to this many tokens the expert stages run fused in one launch
// (k_experts_decode); above it as gate/up, down and combine launches (the
// fused items' handoffs cost more than the two launches they save)
#ifndef FUSED_EXPERTS_MAX_T
#define FUSED_EXPERTS_MAX_T 2
#endif
// sync region (int32 words at the start of the workspace, zero between calls):
// the error word, the per-tile and per-(token, slab) counters of the fused
// expert kernel, then the routing kernel's logit slots.  Counters sit
// SY_STRIDE words (256 bytes) apart.
enum { SY_STRIDE = 64, SY_ERR = 0, SY_TILES = SY_STRIDE };
struct DecodeGeom {
  int nw;                  // waves per expert workgroup
  int wk_gu, wr_gu, wk_dn, wr_dn;
  int slabs_gu, slabs_dn;  // row slabs per tile
  size_t lds;              // dynamic LDS bytes
};
// W4A8 GEMV numerics (moe_w4a8.hip)
// The MoE layer in W4A8: the grouped expert GEMVs over dispatch tiles of at
// most W8_MT tokens and the fp32 combine.
constexpr int W8_MT = 16;
struct W4A8Args {
  const uint8_t *w0, *w1, *ws0, *ws1;     // MODE 0: gate, up; MODE 1: down (w0/ws0)
  const uint16_t *s0, *s1, *ss0, *ss1;
  const int8_t *xq;                      // [T][H] x quantized
  const float *xs;                       // [T][H/128]
  float *act, *act_s;                    // MODE 0 out: [T*k][I], [T][Is]
  const int8_t *aq, *aq_s;               // MODE 1 in: act quantized
  const float *as, *as_s;                // their group scales
  float *o;                              // MODE 1 out: [T*k + T][H]
  const int32_t *ptok;
  const int4 *tiles;
  const int32_t *n_tiles;
  int T, k, E, H, I, Is;
  // MODE 1: act / act_s are the fp32 inputs; the launch quantizes them into
  // aq / as (one token per tile: inside the GEMV kernel, each block into its
  // LDS; else a quantization launch first)
  int quant_in;
};
hipError_t launch_w4a8_expert(int mode, int scale_dtype, const W4A8Args &a, int max_tiles,
                              hipStream_t s);
hipError_t launch_combine_f32(const float *o, const int32_t *inv, const float *w,
                              const float *sg, int has_shared, const void *resid, void *y, int T,
                              int k, int H, const int32_t *err, hipStream_t s);
hipError_t launch_act_quant_i8(const void *x, int x_dtype, int T, int K, int8_t *q, float *sq,
                               hipStream_t s);
// two fp32 quantizations in one launch (x2 may be null)
hipError_t launch_act_quant_f32_pair(const float *x, int T, int K, int8_t *q, float *sq,
                                     const float *x2, int T2, int K2, int8_t *q2, float *sq2,
                                     hipStream_t s);
hipError_t launch_int4_gemv_i8(const uint8_t *P, const void *S, int scale_dtype, const int8_t *xq,
                               const float *sq, int M, int K, int T, float *y, hipStream_t s);
// 0 when the shape has no decode geometry (the staged path is used then)
int decode_geometry(const ainfer_moe_shape &s, DecodeGeom *g);
// router logits + top-k + weights + shared gate + x in MFMA order, and the
// dispatch (tiles of DEC_MT tokens) when ds != NULL
hipError_t launch_route_decode(const void *x, const void *rw, const float *bias, const void *gw,
                               float *logits, float *sgl, int32_t *idx, float *w, float *sg,
                               void *xperm, int T, int H, int E, int k, int has_shared,
                               const DispatchOut *ds, int32_t *sync, uint32_t *slots,
                               const NormIn *norm, hipStream_t s, int8_t *w8q = nullptr,
                               float *w8sq = nullptr);
// gate/up + SiLU, down and the combine (y = sum_j w_j o_j + g_s o_s (+ resid));
// split: gate/up in a launch of its own first (measured faster at T = 1,
// where the down items of a fused launch wait behind the gate/up items for
// workgroup slots: c3 39.5 -> 33.0 us, c1 equal)
// (split: only the down items and the combine; the caller has launched the
// gate/up items, k_expert_lds, just before)
hipError_t launch_experts_decode(int scale_dtype, const DecodeGeom &g, ExpertArgs gu,
                                 ExpertArgs dn, const float *w, const float *sg,
                                 const int32_t *inv, const void *resid, void *y,
                                 int32_t *sync, int max_tiles, int cap, bool split,
                                 hipStream_t s);
hipError_t launch_zero_i32(int32_t *p, int n, hipStream_t s);

// k-groups per wave of the 4-token down items: whole 256-byte row segments
// once the down K (the intermediate size) has 8 groups or more
#ifndef DOWN_KBW4_MIN_I
#define DOWN_KBW4_MIN_I 1024  // c3 T=64: down 149.5 -> 139.5 us; c1 (I = 512) keeps 2
#endif
inline int down_kbw_of(const ainfer_moe_shape &s) {
  const int I = s.inter > s.shared_inter ? s.inter : s.shared_inter;
  return I >= DOWN_KBW4_MIN_I ? 4 : DEC_KBW_DOWN;
}

// ---- persistent decode stack (moe_stack.hip) ------------------------------
// One entry of the device layer table (ainfer_moe_stack_prepare).
struct StackLayer {
  ainfer_moe_weights w;
  const void *norm_w;  // RMSNorm weight [H] bf16, or null (unit)
  const void *pad;
};
struct StackGeom {
  int nw, wk_gu, wr_gu, wk_dn, wr_dn, kbw_dn, slabs_gu, slabs_dn;
  size_t lds;
};
// The stack kernel's workspace pieces: its counters and item flags (in the
// zeroed head of the workspace) and the per-layer regions.
struct StackWs {
  int32_t *flags;    // stack_flag_words
  int cap;           // tile capacity of the item flag arrays
  uint8_t *layers;   // n_layers regions of stack_layer_bytes(T)
  int32_t *err;
};
// bytes of one layer's region at T tokens (offs: the 6 piece offsets)
size_t stack_layer_bytes(const ainfer_moe_shape &s, int T, size_t *offs);
// false when the shape has no stack geometry at T tokens (use block_forward)
bool stack_geometry(const ainfer_moe_shape &s, int T, StackGeom *g);
int stack_flag_words(const ainfer_moe_shape &s, int cap);
hipError_t launch_decode_stack(int scale_dtype, const ainfer_moe_shape &s, const StackGeom &g,
                               const StackLayer *layers, int L, const void *x0, void *r, int T,
                               int norm_mode, float eps, const StackWs &w, hipStream_t st);
