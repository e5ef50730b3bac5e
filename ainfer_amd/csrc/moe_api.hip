// moe_api.hip - the C ABI of include/ainfer_moe.h: validation, workspace
// layout and the stage sequence router -> top-k -> dispatch -> gate/up ->
// down -> combine.  Host code; every device buffer comes from the caller.
#include <string.h>

#include <atomic>
#include <map>
#include <mutex>
#include <vector>

#include "moe_common.h"
#include "moe_internal.h"

namespace {

// ---- profiling: one event per stage boundary, per call ---------------------
constexpr int NSTAGE = AINFER_MOE_N_STAGES;
constexpr int PROF_SLOTS = 64;
struct Prof {
  bool on = false;
  bool created = false;
  hipEvent_t ev[PROF_SLOTS][NSTAGE + 1];
  bool used[PROF_SLOTS][NSTAGE + 1];
  int slot = 0, calls = 0;
  double sum_us[NSTAGE];
  int cnt[NSTAGE];
  // the decode gate/up kernel's own start and end (hipExtLaunchKernel events,
  // stamped by the dispatch: no barrier packets of their own)
  hipEvent_t kev[PROF_SLOTS][2];
  bool kused[PROF_SLOTS];
  double ksum_us;
  int kcnt;
} g_prof;

void prof_flush_slot(int s) {
  // stage i spans the last recorded event before it to its own end event
  int prev = -1;
  for (int i = 0; i <= NSTAGE; ++i) {
    if (!g_prof.used[s][i]) continue;
    if (prev >= 0) {
      (void)hipEventSynchronize(g_prof.ev[s][i]);
      float ms = 0.f;
      if (hipEventElapsedTime(&ms, g_prof.ev[s][prev], g_prof.ev[s][i]) == hipSuccess) {
        g_prof.sum_us[i - 1] += ms * 1000.0;
        g_prof.cnt[i - 1] += 1;
      }
    }
    prev = i;
    g_prof.used[s][i] = false;
  }
  if (g_prof.kused[s]) {
    float ms = 0.f;
    if (hipEventSynchronize(g_prof.kev[s][1]) == hipSuccess &&
        hipEventElapsedTime(&ms, g_prof.kev[s][0], g_prof.kev[s][1]) == hipSuccess) {
      g_prof.ksum_us += ms * 1000.0;
      g_prof.kcnt += 1;
    }
    g_prof.kused[s] = false;
  }
}

struct ProfCall {
  int s = -1;
  hipStream_t st;
  explicit ProfCall(hipStream_t stream) : st(stream) {
    if (!g_prof.on) return;
    s = g_prof.slot;
    g_prof.slot = (g_prof.slot + 1) % PROF_SLOTS;
    prof_flush_slot(s);  // reuse: collect the slot's previous call first
    g_prof.calls++;
  }
  // mark the end of stage `stage` (index = stage + 1); the call's first
  // mark is the start event
  void start() {
    if (s >= 0) rec(0);
  }
  void end(int stage) {
    if (s >= 0) rec(stage + 1);
  }
  void rec(int i) {
    (void)hipEventRecord(g_prof.ev[s][i], st);
    g_prof.used[s][i] = true;
  }
  // the next gate/up expert launch records its own start and end
  void kernel_events() {
    if (s < 0) return;
    set_expert_launch_events(g_prof.kev[s][0], g_prof.kev[s][1]);
    g_prof.kused[s] = true;
  }
};

struct Layout {
  size_t w8_xq, w8_xs, w8_act, w8_acts, w8_aq, w8_as, w8_aqs, w8_ass, w8_o;
  size_t stack_flags, stack_cap, stack_end;
  size_t sync, sync_words, slots, tiles2, n_tiles2, logits, sg_logit, idx, w, sg, xperm, chunk_counts, chunk_masks, rank, counts, offsets, perm, inv,
      ptok, tiles, n_tiles, ticket, act, act_s, o, h, wnorm, xsum, asum, asum_s, total;
};

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// Tiles of at most mt rows over the experts a step selects: sum_e
// ceil(c_e / mt) <= (T*k + (mt - 1) * min(T*k, E)) / mt, plus the shared
// expert's ceil(T / mt).
int max_tiles_bound(const ainfer_moe_shape &s, int T, int mt) {
  long tk = (long)T * s.top_k;
  long used = tk < s.n_experts ? tk : s.n_experts;
  long routed = (tk + (mt - 1) * used + mt - 1) / mt;
  long sh = s.shared_inter > 0 ? (T + mt - 1) / mt : 0;
  return (int)(routed + sh);
}

Layout layout_of(const ainfer_moe_shape &s, int Tm) {
  Layout L;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    size_t o = off;
    off += align256(bytes);
    return o;
  };
  const size_t T = (size_t)(Tm > 0 ? Tm : 1), E = s.n_experts, k = s.top_k, H = s.hidden;
  const size_t nchunks = (T + 63) / 64;
  // decode sync region: the same place and size for every T
  {
    DecodeGeom g;
    const int slabs = decode_geometry(s, &g) ? g.slabs_dn : 0;
    L.slots = SY_TILES + SY_STRIDE * (2 * (size_t)max_tiles_bound(s, DECODE_MAX_T, DEC_MT) +
                                      (size_t)DECODE_MAX_T * slabs);  // in words
    L.sync_words = L.slots + (size_t)DECODE_MAX_T * (E + 1);
    L.sync = take(L.sync_words * 4);
  }
  // the decode-stack kernel's tagged logit slots and item flags: also the
  // same place for every T, zeroed with the sync region
  L.stack_cap = (size_t)max_tiles_bound(s, DECODE_NORM_MAX_T, DEC_MT);
  L.stack_flags = take((size_t)stack_flag_words(s, (int)L.stack_cap) * 4);
  L.stack_end = off;
  L.logits = take(T * E * 4);
  L.sg_logit = take(T * 4);
  L.idx = take(T * k * 4);
  L.w = take(T * k * 4);
  L.sg = take(T * 4);
  L.xperm = take(T * H * 2);
  L.chunk_counts = take(nchunks * E * 4);
  L.chunk_masks = take(nchunks * E * 8);  // right after the counts: zeroed as one range
  L.rank = take(T * k * 4);
  L.counts = take(E * 4);
  L.offsets = take((E + 1) * 4);
  L.perm = take(T * k * 4);
  L.inv = take(T * k * 4);
  L.ptok = take(T * k * 4);
  L.tiles = take((size_t)max_tiles_bound(s, (int)T, DEC_MT) * 16);  // >= every other bound
  L.n_tiles = take(4);
  L.ticket = take(4);
  L.tiles2 = take((E * ((GEMM_SMALL_MAX + SMALL_MT - 1) / SMALL_MT) + 1) * 16);
  L.n_tiles2 = take(4);
  L.act = take(T * k * s.inter * 2);
  L.act_s = take(T * (size_t)(s.shared_inter > 0 ? s.shared_inter : 1) * 2);
  L.o = take(T * (k + 1) * H * 2);
  L.h = take(T * H * 2);
  L.wnorm = take(E * 4);
  L.xsum = take(T * (H / 128) * 4);
  L.asum = take(T * k * (s.inter / 32) * 4);
  L.asum_s = take(T * (size_t)(s.shared_inter > 0 ? s.shared_inter / 32 : 1) * 4);
  L.w8_xq = L.w8_xs = L.w8_act = L.w8_acts = L.w8_aq = L.w8_as = L.w8_aqs = L.w8_ass = L.w8_o = 0;
  if (s.precision == AINFER_PRECISION_W4A8) {
    const size_t Is = s.shared_inter > 0 ? s.shared_inter : 128, I = s.inter;
    L.w8_xq = take(T * H);
    L.w8_xs = take(T * (H / 128) * 4);
    L.w8_act = take(T * k * I * 4);
    L.w8_acts = take(T * Is * 4);
    L.w8_aq = take(T * k * I);
    L.w8_as = take(T * k * (I / 128) * 4);
    L.w8_aqs = take(T * Is);
    L.w8_ass = take(T * (Is / 128) * 4);
    L.w8_o = take(T * (k + 1) * H * 4);
  }
  L.total = off;
  return L;
}

template <typename P>
P *at(void *ws, size_t off) {
  return (P *)((char *)ws + off);
}

// Calls above AINFER_MOE_CHUNK_TOKENS tokens run as consecutive chunks of at
// most that many tokens on one workspace (the chunked prefill of the
// reference's recorded ChunkGemm lists): the workspace and every buffer offset
// stay those of one chunk.  Each token's routing and expert rows are computed
// within its chunk.
constexpr int CHUNK = AINFER_MOE_CHUNK_TOKENS;
int chunk_of(int T) { return T < CHUNK ? T : CHUNK; }

int check_ws(const ainfer_moe_shape *s, int T, void *ws, size_t ws_bytes) {
  if (!ws) return AINFER_ERR_NULL;
  if (((uintptr_t)ws) & 255) return AINFER_ERR_WORKSPACE;
  if (ws_bytes < layout_of(*s, T).total) return AINFER_ERR_WORKSPACE;
  return AINFER_OK;
}

int check_weights(const ainfer_moe_shape *s, const ainfer_moe_weights *w) {
  if (!w || !w->router_w || !w->w_gate || !w->s_gate || !w->w_up || !w->s_up || !w->w_down ||
      !w->s_down)
    return AINFER_ERR_NULL;
  if (s->shared_inter > 0 && (!w->ws_gate || !w->ss_gate || !w->ws_up || !w->ss_up ||
                              !w->ws_down || !w->ss_down))
    return AINFER_ERR_NULL;
  // 16-byte vector loads of weights, 8-byte loads of scale runs
  auto mis = [](const void *p, uintptr_t a) { return p && ((uintptr_t)p & (a - 1)); };
  if (mis(w->w_gate, 16) || mis(w->w_up, 16) || mis(w->w_down, 16) || mis(w->ws_gate, 16) ||
      mis(w->ws_up, 16) || mis(w->ws_down, 16) || mis(w->router_w, 16) ||
      mis(w->shared_gate_w, 16) || mis(w->s_gate, 8) || mis(w->s_up, 8) || mis(w->s_down, 8) ||
      mis(w->ss_gate, 8) || mis(w->ss_up, 8) || mis(w->ss_down, 8))
    return AINFER_ERR_ARG;
  return AINFER_OK;
}

#define HIP_TRY(expr)                              \
  do {                                             \
    if ((expr) != hipSuccess) return AINFER_ERR_HIP; \
  } while (0)
#define HIP_TRY_RC(expr)          \
  do {                            \
    const int rc_ = (expr);       \
    if (rc_ != AINFER_OK) return rc_; \
  } while (0)

DispatchOut dispatch_out(const ainfer_moe_shape *s, const Layout &L, void *ws, int T) {
  DispatchOut d;
  d.counts = at<int32_t>(ws, L.counts);
  d.offsets = at<int32_t>(ws, L.offsets);
  d.perm = at<int32_t>(ws, L.perm);
  d.inv = at<int32_t>(ws, L.inv);
  d.ptok = at<int32_t>(ws, L.ptok);
  d.tiles = at<int4>(ws, L.tiles);
  d.n_tiles = at<int32_t>(ws, L.n_tiles);
  d.ticket = at<int32_t>(ws, L.ticket);
  d.tiles2 = at<int4>(ws, L.tiles2);
  d.n_tiles2 = at<int32_t>(ws, L.n_tiles2);
  d.small_max = 0;
  d.mt = SMALL_MT;
  return d;
}

// Arguments of the small-tile expert kernels: mode 0 = gate/up (+ SiLU), mode
// 1 = down.
ExpertArgs expert_args(const ainfer_moe_shape *s, const ainfer_moe_weights *w, const Layout &L,
                       void *ws, const DispatchOut &d, int T, int mode) {
  ExpertArgs a;
  memset(&a, 0, sizeof a);
  a.ptok = d.ptok;
  a.tiles = d.tiles;
  a.n_tiles = d.n_tiles;
  a.T = T;
  a.k = s->top_k;
  a.E = s->n_experts;
  a.H = s->hidden;
  a.I = s->inter;
  a.Is = s->shared_inter;
  if (mode == 0) {
    a.w0 = w->w_gate;
    a.w1 = w->w_up;
    a.s0 = (const uint16_t *)w->s_gate;
    a.s1 = (const uint16_t *)w->s_up;
    a.ws0 = w->ws_gate;
    a.ws1 = w->ws_up;
    a.ss0 = (const uint16_t *)w->ss_gate;
    a.ss1 = (const uint16_t *)w->ss_up;
    a.a_routed = at<uint16_t>(ws, L.xperm);
    a.a_shared = at<uint16_t>(ws, L.xperm);
    a.act = at<uint16_t>(ws, L.act);
    a.act_s = at<uint16_t>(ws, L.act_s);
  } else {
    a.w0 = w->w_down;
    a.s0 = (const uint16_t *)w->s_down;
    a.ws0 = w->ws_down;
    a.ss0 = (const uint16_t *)w->ss_down;
    a.a_routed = at<uint16_t>(ws, L.act);
    a.a_shared = at<uint16_t>(ws, L.act_s);
    a.o = at<uint16_t>(ws, L.o);
  }
  return a;
}

#ifndef SGU_KBW
#define SGU_KBW 4
#endif
#ifndef SGU_RG
#define SGU_RG RG_GATE_UP
#endif
#ifndef SDN_KBW
#define SDN_KBW 2
#endif
#ifndef SDN_RG
#define SDN_RG RG_DOWN
#endif
// norm (decode path only, ainfer_moe_block_forward): x is the residual stream and
// the routing kernel applies the RMSNorm itself
int down_kbw(const ainfer_moe_shape &s) { return down_kbw_of(s); }

// The layer in W4A8 (AINFER_PRECISION_W4A8): the routing and dispatch of
// the W4A16 path, then x quantized, the grouped gate/up GEMVs with SiLU, act
// quantized, the grouped down GEMVs and the fp32 combine (moe_w4a8.hip).
// Decode sizes take the W4A16 decode routing kernel (canonical logits,
// top-k, weights, gate, the MFMA-order copy of x with its W4A8 codes, the
// dispatch in tiles of DEC_MT tokens, and with norm the block's RMSNorm);
// larger T the staged router, 16-token tiles and x quantized on its own.
int do_forward_w4a8(const ainfer_moe_shape *s, const ainfer_moe_weights *w, const void *x,
                    const void *resid, void *y, int T, void *ws, hipStream_t st, ProfCall *pc,
                    const NormIn *norm = nullptr) {
  const Layout L = layout_of(*s, T);
  const int E = s->n_experts, k = s->top_k, H = s->hidden, I = s->inter, Is = s->shared_inter;
  const int has_shared = Is > 0;
  DispatchOut d = dispatch_out(s, L, ws, T);
  const bool decode = T <= DECODE_MAX_T && E <= 1024 && (!norm || T <= DECODE_NORM_MAX_T);
  if (norm && !decode) return AINFER_ERR_ARG;  // the caller normalizes above that
  d.mt = decode ? DEC_MT : W8_MT;
  if (decode) {
    DispatchOut dr = d;  // nothing here reads the per-expert counts or offsets
    dr.counts = nullptr;
    dr.offsets = nullptr;
    int32_t *sync = at<int32_t>(ws, L.sync);
    HIP_TRY(launch_route_decode(x, w->router_w, w->router_bias, w->shared_gate_w,
                                at<float>(ws, L.logits), at<float>(ws, L.sg_logit),
                                at<int32_t>(ws, L.idx), at<float>(ws, L.w), at<float>(ws, L.sg),
                                at<uint16_t>(ws, L.xperm), T, H, E, k, has_shared, &dr, sync,
                                (uint32_t *)(sync + L.slots), norm, st, at<int8_t>(ws, L.w8_xq),
                                at<float>(ws, L.w8_xs)));
    pc->end(3);
  } else if (T <= EXACT_ROUTER_MAX_T)
    HIP_TRY(launch_router_exact(x, w->router_w, w->router_bias, w->shared_gate_w,
                                at<float>(ws, L.logits), at<float>(ws, L.sg_logit),
                                at<int32_t>(ws, L.idx), at<float>(ws, L.w), at<float>(ws, L.sg),
                                at<uint16_t>(ws, L.xperm), T, H, E, k, has_shared, nullptr, st));
  else
    HIP_TRY(launch_router_fast(x, w->router_w, w->router_bias, w->shared_gate_w,
                               at<float>(ws, L.logits), at<float>(ws, L.wnorm),
                               at<int32_t>(ws, L.idx), at<float>(ws, L.w), at<float>(ws, L.sg),
                               at<uint16_t>(ws, L.xperm), nullptr, T, H, E, k, has_shared,
                               nullptr, st));
  if (!decode) {
    pc->end(2);
    HIP_TRY(launch_dispatch(at<int32_t>(ws, L.idx), T, k, E, W8_MT, has_shared,
                            at<int32_t>(ws, L.chunk_counts), at<int32_t>(ws, L.rank), d, st));
    pc->end(3);
  }
  W4A8Args a;
  memset(&a, 0, sizeof a);
  a.xq = at<int8_t>(ws, L.w8_xq);
  a.xs = at<float>(ws, L.w8_xs);
  a.act = at<float>(ws, L.w8_act);
  a.act_s = at<float>(ws, L.w8_acts);
  a.aq = at<int8_t>(ws, L.w8_aq);
  a.as = at<float>(ws, L.w8_as);
  a.aq_s = at<int8_t>(ws, L.w8_aqs);
  a.as_s = at<float>(ws, L.w8_ass);
  a.o = at<float>(ws, L.w8_o);
  a.ptok = d.ptok;
  a.tiles = d.tiles;
  a.n_tiles = d.n_tiles;
  a.T = T;
  a.k = k;
  a.E = E;
  a.H = H;
  a.I = I;
  a.Is = Is;
  const int mtb = max_tiles_bound(*s, T, d.mt);
  if (!decode)  // the decode routing kernel wrote the codes with its x copy
    HIP_TRY(launch_act_quant_i8(x, AINFER_ACT_BF16, T, H, at<int8_t>(ws, L.w8_xq),
                                at<float>(ws, L.w8_xs), st));
  a.w0 = w->w_gate;
  a.w1 = w->w_up;
  a.s0 = (const uint16_t *)w->s_gate;
  a.s1 = (const uint16_t *)w->s_up;
  a.ws0 = w->ws_gate;
  a.ws1 = w->ws_up;
  a.ss0 = (const uint16_t *)w->ss_gate;
  a.ss1 = (const uint16_t *)w->ss_up;
  HIP_TRY(launch_w4a8_expert(0, s->scale_dtype, a, mtb, st));
  pc->end(4);
  // the down launch quantizes act itself (at T = 1 inside its blocks)
  a.quant_in = 1;
  a.w0 = w->w_down;
  a.s0 = (const uint16_t *)w->s_down;
  a.ws0 = w->ws_down;
  a.ss0 = (const uint16_t *)w->ss_down;
  a.w1 = a.ws1 = nullptr;
  a.s1 = a.ss1 = nullptr;
  HIP_TRY(launch_w4a8_expert(1, s->scale_dtype, a, mtb, st));
  pc->end(5);
  HIP_TRY(launch_combine_f32(a.o, d.inv, at<float>(ws, L.w), at<float>(ws, L.sg), has_shared,
                             resid, y, T, k, H, at<int32_t>(ws, L.sync) + SY_ERR, st));
  pc->end(6);
  return AINFER_OK;
}

// The expert stage on the dispatch d in the workspace, x in MFMA order
// written (and its group sums at T >= GEMM_MIN_T): the grouped GEMM there
// (with the small experts' 16-token tiles), else the streaming items over
// tiles of DEC_MT tokens.  Leaves o in the workspace: dispatch-position rows,
// the shared expert's at rows T * k + t.
int run_experts(const ainfer_moe_shape *s, const ainfer_moe_weights *w, const Layout &L,
                void *ws, DispatchOut &d, int T, bool gemm, hipStream_t st, ProfCall *pc) {
  const int E = s->n_experts, k = s->top_k, H = s->hidden;
  if (gemm) {
    GemmArgs g;
    memset(&g, 0, sizeof g);
    g.ptok = d.ptok;
    g.tiles = d.tiles;
    g.n_tiles = d.n_tiles;
    g.T = T;
    g.k = k;
    g.E = E;
    g.H = H;
    g.I = s->inter;
    g.Is = s->shared_inter;
    g.xsum = at<float>(ws, L.xsum);
    g.asum = at<float>(ws, L.asum);
    g.asum_s = at<float>(ws, L.asum_s);
    const int gtiles = max_tiles_bound(*s, T, GEMM_MT);
    g.w0 = w->w_gate;
    g.w1 = w->w_up;
    g.s0 = (const uint16_t *)w->s_gate;
    g.s1 = (const uint16_t *)w->s_up;
    g.ws0 = w->ws_gate;
    g.ws1 = w->ws_up;
    g.ss0 = (const uint16_t *)w->ss_gate;
    g.ss1 = (const uint16_t *)w->ss_up;
    g.a_routed = at<uint16_t>(ws, L.xperm);
    g.act = at<uint16_t>(ws, L.act);
    g.act_s = at<uint16_t>(ws, L.act_s);
    HIP_TRY(launch_expert_gemm(0, s->scale_dtype, g, gtiles, st));
    ExpertArgs sgu, sdn;
    int small_bound = 0;
    if (d.small_max > 0) {
      DispatchOut d2 = d;
      d2.tiles = d.tiles2;
      d2.n_tiles = d.n_tiles2;
      sgu = expert_args(s, w, L, ws, d2, T, 0);
      sdn = expert_args(s, w, L, ws, d2, T, 1);
      // tiles2 holds at most E * ceil(small_max / SMALL_MT) tiles, and at
      // most one partial tile per expert beyond T * k / SMALL_MT full ones
      const long b1 = (long)E * ((GEMM_SMALL_MAX + SMALL_MT - 1) / SMALL_MT);
      const long b2 = (long)T * k / SMALL_MT + E;
      small_bound = (int)(b1 < b2 ? b1 : b2);
      HIP_TRY(launch_expert_stream(0, s->scale_dtype, sgu, small_bound, SGU_KBW, SGU_RG, SMALL_MT,
                                   st));
    }
    pc->end(4);
    g.w0 = w->w_down;
    g.s0 = (const uint16_t *)w->s_down;
    g.ws0 = w->ws_down;
    g.ss0 = (const uint16_t *)w->ss_down;
    g.w1 = nullptr;
    g.s1 = nullptr;
    g.ws1 = nullptr;
    g.ss1 = nullptr;
    g.a_routed = at<uint16_t>(ws, L.act);
    g.a_shared = at<uint16_t>(ws, L.act_s);
    g.o = at<uint16_t>(ws, L.o);
    HIP_TRY(launch_expert_gemm(1, s->scale_dtype, g, gtiles, st));
    if (d.small_max > 0) {
      HIP_TRY(launch_expert_stream(1, s->scale_dtype, sdn, small_bound, SDN_KBW, SDN_RG, SMALL_MT,
                                   st));
    }
    pc->end(5);
    return AINFER_OK;
  }
  ExpertArgs a;
  memset(&a, 0, sizeof a);
  a.ptok = d.ptok;
  a.tiles = d.tiles;
  a.n_tiles = d.n_tiles;
  a.T = T;
  a.k = k;
  a.E = E;
  a.H = H;
  a.I = s->inter;
  a.Is = s->shared_inter;
  const int smt = DEC_MT;  // tiles of the dispatch above
  const int max_tiles = max_tiles_bound(*s, T, smt);
  // k-groups per wave and 16-row groups per wave, measured at T = 1, 4, 16
  const int kbw = 4, kbw_down = down_kbw(*s);
  // gate/up + SiLU-mul
  a.w0 = w->w_gate;
  a.w1 = w->w_up;
  a.s0 = (const uint16_t *)w->s_gate;
  a.s1 = (const uint16_t *)w->s_up;
  a.ws0 = w->ws_gate;
  a.ws1 = w->ws_up;
  a.ss0 = (const uint16_t *)w->ss_gate;
  a.ss1 = (const uint16_t *)w->ss_up;
  a.a_routed = at<uint16_t>(ws, L.xperm);
  a.a_shared = at<uint16_t>(ws, L.xperm);
  a.act = at<uint16_t>(ws, L.act);
  a.act_s = at<uint16_t>(ws, L.act_s);
  HIP_TRY(launch_expert_stream(0, s->scale_dtype, a, max_tiles, kbw, RG_GATE_UP, smt, st));
  pc->end(4);
  // down + combine
  a.w0 = w->w_down;
  a.s0 = (const uint16_t *)w->s_down;
  a.ws0 = w->ws_down;
  a.ss0 = (const uint16_t *)w->ss_down;
  a.w1 = nullptr;
  a.s1 = nullptr;
  a.ws1 = nullptr;
  a.ss1 = nullptr;
  a.a_routed = at<uint16_t>(ws, L.act);
  a.a_shared = at<uint16_t>(ws, L.act_s);
  a.o = at<uint16_t>(ws, L.o);
  HIP_TRY(launch_expert_stream(1, s->scale_dtype, a, max_tiles, kbw_down, RG_DOWN, smt, st));
  pc->end(5);
  return AINFER_OK;
}

int do_forward(const ainfer_moe_shape *s, const ainfer_moe_weights *w, const void *x,
               const void *resid, void *y, int T, void *ws, hipStream_t st,
               ProfCall *pc, const NormIn *norm = nullptr, const NormIn *next = nullptr,
               void *h_next = nullptr) {
  // the final combine, or (next non-null, W4A16, resid non-null) the combine
  // followed by the next block's RMSNorm of the rows it writes, into h_next
  auto combine = [&](const DispatchOut &d, const Layout &L) -> hipError_t {
    if (next && resid)
      return launch_combine_norm(at<uint16_t>(ws, L.o), d.inv, at<float>(ws, L.w),
                                 at<float>(ws, L.sg), s->shared_inter > 0, resid, y, T,
                                 s->top_k, s->hidden, at<int32_t>(ws, L.sync) + SY_ERR, *next,
                                 h_next, st);
    return launch_combine(at<uint16_t>(ws, L.o), d.inv, at<float>(ws, L.w), at<float>(ws, L.sg),
                          s->shared_inter > 0, resid, y, T, s->top_k, s->hidden,
                          at<int32_t>(ws, L.sync) + SY_ERR, st);
  };
  if (s->precision == AINFER_PRECISION_W4A8)
    return do_forward_w4a8(s, w, x, resid, y, T, ws, st, pc, norm);
  const Layout L = layout_of(*s, T);
  const int E = s->n_experts, k = s->top_k, H = s->hidden;
  const int has_shared = s->shared_inter > 0;
  const bool fused = T <= FUSED_DISPATCH_MAX_T;
  const bool gemm = T >= GEMM_MIN_T;
  // below GEMM_MIN_T most experts get at most 4 tokens: tiles of DEC_MT for
  // the LDS-staged items (c3 T=64: 629 -> 477 us against 16-token tiles)
  const int mt = gemm ? GEMM_MT : DEC_MT;
  DispatchOut d = dispatch_out(s, L, ws, T);
  d.mt = mt;
  DecodeGeom dg;
  if (T <= DECODE_MAX_T && decode_geometry(*s, &dg)) {
    // decode: two launches (moe_decode.hip)
    int32_t *sync = at<int32_t>(ws, L.sync);
    // the expert kernels read the tiles and positions only: no per-expert
    // counts or offsets on this path
    DispatchOut dr = d;
    dr.counts = nullptr;
    dr.offsets = nullptr;
    HIP_TRY(launch_route_decode(x, w->router_w, w->router_bias, w->shared_gate_w,
                                at<float>(ws, L.logits), at<float>(ws, L.sg_logit),
                                at<int32_t>(ws, L.idx), at<float>(ws, L.w), at<float>(ws, L.sg),
                                at<uint16_t>(ws, L.xperm), T, H, E, k, has_shared, &dr, sync,
                                (uint32_t *)(sync + L.slots), norm, st));
    pc->end(2);
    ExpertArgs gu = expert_args(s, w, L, ws, d, T, 0), dn = expert_args(s, w, L, ws, d, T, 1);
    if (T <= FUSED_EXPERTS_MAX_T) {
      // latency-bound: gate/up, down and combine in one launch (T = 1: the
      // gate/up items in a launch of their own first)
      if (T == 1) {
        pc->kernel_events();
        HIP_TRY(launch_expert_stream(0, s->scale_dtype, gu, max_tiles_bound(*s, T, DEC_MT), 4,
                                     DEC_RG_GATE_UP, DEC_MT, st));
        pc->end(4);
      }
      HIP_TRY(launch_experts_decode(s->scale_dtype, dg, gu, dn, at<float>(ws, L.w),
                                    at<float>(ws, L.sg), d.inv, resid, y, sync,
                                    max_tiles_bound(*s, T, DEC_MT),
                                    max_tiles_bound(*s, DECODE_MAX_T, DEC_MT), T == 1, st));
    } else {
      // bandwidth-bound: three launches whose items hold no waits
      const int mtb = max_tiles_bound(*s, T, DEC_MT);
      pc->kernel_events();
      HIP_TRY(launch_expert_stream(0, s->scale_dtype, gu, mtb, 4, DEC_RG_GATE_UP, DEC_MT, st));
      pc->end(4);
      HIP_TRY(launch_expert_stream(1, s->scale_dtype, dn, mtb, down_kbw(*s), DEC_RG_DOWN, DEC_MT, st));
      pc->end(5);
      HIP_TRY(combine(d, L));
      pc->end(6);
      return AINFER_OK;
    }
    pc->end(5);
    return AINFER_OK;
  }
  if (T <= EXACT_ROUTER_MAX_T)
    HIP_TRY(launch_router_exact(x, w->router_w, w->router_bias, w->shared_gate_w,
                                at<float>(ws, L.logits), at<float>(ws, L.sg_logit),
                                at<int32_t>(ws, L.idx), at<float>(ws, L.w), at<float>(ws, L.sg),
                                at<uint16_t>(ws, L.xperm), T, H, E, k, has_shared,
                                fused ? &d : nullptr, st));
  // prefill (T >= GEMM_MIN_T, unfused dispatch): the selection builds the
  // dispatch's per-chunk token masks itself, so the dispatch needs no counting launch
  unsigned long long *cmask =
      gemm && !fused ? at<unsigned long long>(ws, L.chunk_masks) : nullptr;
  if (T > EXACT_ROUTER_MAX_T)
    HIP_TRY(launch_router_fast(x, w->router_w, w->router_bias, w->shared_gate_w,
                               at<float>(ws, L.logits), at<float>(ws, L.wnorm),
                               at<int32_t>(ws, L.idx), at<float>(ws, L.w), at<float>(ws, L.sg),
                               at<uint16_t>(ws, L.xperm), gemm ? at<float>(ws, L.xsum) : nullptr,
                               T, H, E, k, has_shared, fused ? &d : nullptr, st,
                               cmask ? at<int32_t>(ws, L.chunk_counts) : nullptr, cmask));
  pc->end(2);
  // prefill: experts with at most SMALL_MT tokens skip the GEMM (a 128-token
  // tile costs about half a full one however few tokens it holds) for one
  // 16-token tile of the streaming kernels, which read their weights once
  if (gemm) d.small_max = GEMM_SMALL_MAX;
  if (!fused)
    HIP_TRY(launch_dispatch(at<int32_t>(ws, L.idx), T, k, E, mt, has_shared,
                            at<int32_t>(ws, L.chunk_counts), at<int32_t>(ws, L.rank), d, st,
                            cmask));
  pc->end(3);
  HIP_TRY_RC(run_experts(s, w, L, ws, d, T, gemm, st, pc));
  HIP_TRY(combine(d, L));
  pc->end(6);
  return AINFER_OK;
}

int check_block_args(const ainfer_moe_shape *s, const ainfer_moe_weights *w, int norm_mode,
                     float eps, const void *resid_in, const void *resid_out, int T) {
  int rc = ainfer_moe_validate(s);
  if (rc) return rc;
  if (T < 0 || T > AINFER_MOE_MAX_TOKENS) return AINFER_ERR_TOKENS;
  if ((rc = check_weights(s, w))) return rc;
  if (norm_mode != AINFER_NORM_PLAIN && norm_mode != AINFER_NORM_ONE_PLUS) return AINFER_ERR_ARG;
  if (!(eps >= 0.0f)) return AINFER_ERR_ARG;
  if (T == 0) return AINFER_OK;
  if (!resid_in || !resid_out) return AINFER_ERR_NULL;
  return AINFER_OK;
}

// h = RMSNorm(resid_in); resid_out = resid_in + MoE(h), on a checked workspace
int do_block(const ainfer_moe_shape *s, const ainfer_moe_weights *w, const void *norm_w,
             int norm_mode, float eps, const void *resid_in, void *resid_out, int T, void *ws,
             hipStream_t st) {
  const Layout L = layout_of(*s, T);
  void *h = at<void>(ws, L.h);
  ProfCall pc(st);
  pc.start();
  DecodeGeom dg;
  if (T <= DECODE_NORM_MAX_T && s->n_experts <= 1024 &&
      (s->precision == AINFER_PRECISION_W4A8 || decode_geometry(*s, &dg))) {
    // decode at up to 4 tokens: the routing kernel normalizes x itself (one
    // launch fewer per block: c4 T=1 about 2470 -> 2235 us per 60-block
    // step); the values are those k_rmsnorm writes
    NormIn n;
    n.w = (const uint16_t *)norm_w;
    n.mode = norm_mode;
    n.eps = eps;
    n.on = 1;
    pc.end(0);
    return do_forward(s, w, resid_in, resid_in, resid_out, T, ws, st, &pc, &n);
  }
  HIP_TRY(launch_rmsnorm(resid_in, norm_w, norm_mode, eps, h, T, s->hidden, st));
  pc.end(0);
  return do_forward(s, w, h, resid_in, resid_out, T, ws, st, &pc);
}

// ---- the no-allocation entry's scratch ---------------------------------------
// One copy per GPU, alive until the process ends.  Host code must never pass
// the array's name to a kernel or a copy (on the host it is only a stand-in
// symbol); it uses the per-device address hipGetSymbolAddress returns.
__device__ __align__(256) unsigned char scratch[AINFER_MOE_NOALLOC_SCRATCH_BYTES];

// host copies of the tables ainfer_moe_stack_prepare wrote, by device address
std::mutex g_tables_mu;
std::map<const void *, std::vector<StackLayer>> g_tables;

constexpr int NOALLOC_MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[NOALLOC_MAX_DEVICES];

// The current device's scratch address, looked up once per device.
int noalloc_scratch(void **out) {
  int dev = -1;
  HIP_TRY(hipGetDevice(&dev));
  if (dev < 0 || dev >= NOALLOC_MAX_DEVICES) return AINFER_ERR_HIP;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void *p = nullptr;
    HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p || ((uintptr_t)p & 255)) return AINFER_ERR_HIP;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return AINFER_OK;
}

}  // namespace

namespace {
int do_route(const ainfer_moe_shape *s, const ainfer_moe_weights *w, const void *x, int T,
             int32_t *topk_idx, float *topk_w, float *shared_gate, float *logits, void *ws,
             hipStream_t st) {
  const Layout L = layout_of(*s, T);
  DecodeGeom dg;
  if (T <= DECODE_MAX_T && decode_geometry(*s, &dg)) {
    // the decode routing kernel, without its dispatch
    HIP_TRY(launch_route_decode(x, w->router_w, w->router_bias, w->shared_gate_w,
                                logits ? logits : at<float>(ws, L.logits),
                                at<float>(ws, L.sg_logit), topk_idx, topk_w, shared_gate, nullptr,
                                T, s->hidden, s->n_experts, s->top_k, s->shared_inter > 0,
                                nullptr, at<int32_t>(ws, L.sync),
                                at<uint32_t>(ws, L.sync) + L.slots, nullptr, st));
    return AINFER_OK;
  }
  if (T <= EXACT_ROUTER_MAX_T) {
    HIP_TRY(launch_router_exact(x, w->router_w, w->router_bias, w->shared_gate_w,
                                logits ? logits : at<float>(ws, L.logits),
                                at<float>(ws, L.sg_logit), topk_idx, topk_w, shared_gate, nullptr,
                                T, s->hidden, s->n_experts, s->top_k, s->shared_inter > 0,
                                nullptr, st));
    return AINFER_OK;
  }
  HIP_TRY(launch_router_fast(x, w->router_w, w->router_bias, w->shared_gate_w,
                             at<float>(ws, L.logits), at<float>(ws, L.wnorm), topk_idx, topk_w,
                             shared_gate, nullptr, nullptr, T, s->hidden, s->n_experts,
                             s->top_k, s->shared_inter > 0, nullptr, st));
  // the full canonical logits, on request (lane-strided chunk order, VALU)
  if (logits)
    HIP_TRY(launch_router(x, w->router_w, w->router_bias, w->shared_gate_w, logits,
                          at<float>(ws, L.sg_logit), nullptr, T, s->hidden, s->n_experts, st));
  return AINFER_OK;
}
}  // namespace

extern "C" {

const char *ainfer_moe_strerror(int status) {
  switch (status) {
  case AINFER_OK: return "ok";
  case AINFER_ERR_SHAPE: return "unsupported shape";
  case AINFER_ERR_NULL: return "required pointer is NULL";
  case AINFER_ERR_WORKSPACE: return "workspace too small or not 256-byte aligned";
  case AINFER_ERR_TOKENS: return "token count out of range";
  case AINFER_ERR_HIP: return "HIP runtime error";
  case AINFER_ERR_ARG: return "argument out of range";
  case AINFER_ERR_SYNC: return "a device-side wait ran out (workspace synchronisation words)";
  case AINFER_ERR_SCRATCH:
    return "the call needs more workspace than the no-allocation entry's static scratch holds";
  default: return "unknown status";
  }
}

int ainfer_moe_validate(const ainfer_moe_shape *s) {
  if (!s) return AINFER_ERR_NULL;
  if (s->group != 128) return AINFER_ERR_SHAPE;
  if (s->precision != AINFER_PRECISION_W4A16 && s->precision != AINFER_PRECISION_W4A8)
    return AINFER_ERR_SHAPE;
  // K of every expert product <= 4096 (the prefill GEMM's tables hold 32 groups)
  if (s->hidden < 128 || s->hidden % 128 || s->hidden > 4096) return AINFER_ERR_SHAPE;
  if (s->inter < 128 || s->inter % 128 || s->inter > 4096) return AINFER_ERR_SHAPE;
  if (s->shared_inter < 0 || s->shared_inter % 128 || s->shared_inter > 4096)
    return AINFER_ERR_SHAPE;
  if (s->n_experts < 1 || s->n_experts > 1024) return AINFER_ERR_SHAPE;
  if (s->top_k < 1 || s->top_k > 32 || s->top_k > s->n_experts) return AINFER_ERR_SHAPE;
  if (s->scale_dtype != AINFER_SCALE_FP16 && s->scale_dtype != AINFER_SCALE_BF16)
    return AINFER_ERR_SHAPE;
  if (!router_supported(s->hidden, s->n_experts)) return AINFER_ERR_SHAPE;
  int kbw, wk, wr;
  for (int mode = 0; mode < 2; ++mode)
    if (!expert_geometry(mode, s->hidden, s->inter, s->shared_inter, 1, &kbw, &wk, &wr))
      return AINFER_ERR_SHAPE;
  return AINFER_OK;
}

size_t ainfer_moe_workspace_bytes(const ainfer_moe_shape *s, int32_t max_tokens) {
  if (ainfer_moe_validate(s) != AINFER_OK) return 0;
  if (max_tokens < 0 || max_tokens > AINFER_MOE_MAX_TOKENS) return 0;
  return layout_of(*s, chunk_of(max_tokens)).total;
}

int ainfer_moe_workspace_init(const ainfer_moe_shape *s, void *ws, size_t ws_bytes,
                              void *stream) {
  int rc = ainfer_moe_validate(s);
  if (rc) return rc;
  if ((rc = check_ws(s, 0, ws, ws_bytes))) return rc;
  const Layout L = layout_of(*s, 0);
  HIP_TRY(launch_zero_i32(at<int32_t>(ws, L.sync), (int)((L.stack_end - L.sync) / 4),
                          (hipStream_t)stream));
  return AINFER_OK;
}

int ainfer_moe_workspace_check(const ainfer_moe_shape *s, const void *ws, size_t ws_bytes,
                               void *stream) {
  int rc = ainfer_moe_validate(s);
  if (rc) return rc;
  if ((rc = check_ws(s, 0, const_cast<void *>(ws), ws_bytes))) return rc;
  const Layout L = layout_of(*s, 0);
  std::vector<int32_t> h(L.sync_words);
  HIP_TRY(hipStreamSynchronize((hipStream_t)stream));
  HIP_TRY(hipMemcpy(h.data(), at<int32_t>(const_cast<void *>(ws), L.sync), L.sync_words * 4,
                    hipMemcpyDeviceToHost));
  if (h[SY_ERR]) return AINFER_ERR_SYNC;
  for (size_t i = 0; i < h.size(); ++i)
    if (h[i]) return AINFER_ERR_WORKSPACE;
  return AINFER_OK;
}

}  // extern "C"

namespace {
std::atomic<int> g_strict{0};

// Strict mode: wait for the call's work and report a bounded wait that ran
// out (the workspace's sticky error word).  rc: the call's own result so far.
int strict_finish(int rc, const void *ws, void *stream) {
  if (rc || !g_strict.load() || !ws) return rc;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  HIP_TRY(hipStreamIsCapturing((hipStream_t)stream, &cs));
  if (cs != hipStreamCaptureStatusNone) return AINFER_OK;
  HIP_TRY(hipStreamSynchronize((hipStream_t)stream));
  int32_t err = 0;
  // the sync region starts the workspace (layout_of: offset 0)
  HIP_TRY(hipMemcpy(&err, (const int32_t *)ws + SY_ERR, sizeof err, hipMemcpyDeviceToHost));
  return err ? AINFER_ERR_SYNC : AINFER_OK;
}
}  // namespace

extern "C" {

int ainfer_moe_set_strict(int32_t on) {
  g_strict.store(on ? 1 : 0);
  return AINFER_OK;
}

int ainfer_moe_forward(const ainfer_moe_shape *s, const ainfer_moe_weights *w, const void *x,
                       void *y, int32_t T, void *ws, size_t ws_bytes, void *stream) {
  int rc = ainfer_moe_validate(s);
  if (rc) return rc;
  if (T < 0 || T > AINFER_MOE_MAX_TOKENS) return AINFER_ERR_TOKENS;
  if ((rc = check_weights(s, w))) return rc;
  if (T == 0) return AINFER_OK;
  if (!x || !y) return AINFER_ERR_NULL;
  if ((rc = check_ws(s, chunk_of(T), ws, ws_bytes))) return rc;
  const size_t row = (size_t)s->hidden * 2;
  for (int t0 = 0; t0 < T; t0 += CHUNK) {
    ProfCall pc((hipStream_t)stream);
    pc.start();
    if ((rc = do_forward(s, w, (const char *)x + t0 * row, nullptr, (char *)y + t0 * row,
                         chunk_of(T - t0), ws, (hipStream_t)stream, &pc)))
      return rc;
  }
  return strict_finish(AINFER_OK, ws, stream);
}

int ainfer_moe_block_forward(const ainfer_moe_shape *s, const ainfer_moe_weights *w,
                             const void *norm_w, int32_t norm_mode, float eps,
                             const void *resid_in, void *resid_out, int32_t T, void *ws,
                             size_t ws_bytes, void *stream) {
  int rc = check_block_args(s, w, norm_mode, eps, resid_in, resid_out, T);
  if (rc || T == 0) return rc;
  if ((rc = check_ws(s, chunk_of(T), ws, ws_bytes))) return rc;
  const size_t row = (size_t)s->hidden * 2;
  for (int t0 = 0; t0 < T; t0 += CHUNK)
    if ((rc = do_block(s, w, norm_w, norm_mode, eps, (const char *)resid_in + t0 * row,
                       (char *)resid_out + t0 * row, chunk_of(T - t0), ws, (hipStream_t)stream)))
      return rc;
  return strict_finish(AINFER_OK, ws, stream);
}

int ainfer_moe_block_forward_noalloc(const ainfer_moe_shape *s, const ainfer_moe_weights *w,
                                     const void *norm_w, int32_t norm_mode, float eps,
                                     const void *resid_in, void *resid_out, int32_t T,
                                     void *stream) {
  int rc = check_block_args(s, w, norm_mode, eps, resid_in, resid_out, T);
  if (rc || T == 0) return rc;
  if (layout_of(*s, chunk_of(T)).total > AINFER_MOE_NOALLOC_SCRATCH_BYTES)
    return AINFER_ERR_SCRATCH;
  void *ws = nullptr;
  if ((rc = noalloc_scratch(&ws))) return rc;
  hipStream_t st = (hipStream_t)stream;
  // every call starts from zeroed synchronisation words (a fill kernel, so the
  // call stays capturable into a HIP graph): a bounded wait that ran out in
  // an earlier call (that call's outputs are NaN) leaves nothing behind
  const Layout L0 = layout_of(*s, 0);
  HIP_TRY(launch_zero_i32(at<int32_t>(ws, L0.sync), (int)L0.sync_words, st));
  const size_t row = (size_t)s->hidden * 2;
  for (int t0 = 0; t0 < T; t0 += CHUNK)
    if ((rc = do_block(s, w, norm_w, norm_mode, eps, (const char *)resid_in + t0 * row,
                       (char *)resid_out + t0 * row, chunk_of(T - t0), ws, st)))
      return rc;
  return strict_finish(AINFER_OK, ws, stream);
}

size_t ainfer_moe_stack_table_bytes(int32_t n_layers) {
  return n_layers > 0 ? (size_t)n_layers * sizeof(StackLayer) : 0;
}

int ainfer_moe_stack_prepare(const ainfer_moe_shape *s, const ainfer_moe_weights *layers,
                             const void *const *norm_w, int32_t n_layers, void *table,
                             size_t table_bytes, void *stream) {
  int rc = ainfer_moe_validate(s);
  if (rc) return rc;
  if (n_layers <= 0) return AINFER_ERR_ARG;
  if (!layers || !table) return AINFER_ERR_NULL;
  if (((uintptr_t)table) & 15 || table_bytes < ainfer_moe_stack_table_bytes(n_layers))
    return AINFER_ERR_ARG;
  std::vector<StackLayer> h((size_t)n_layers);
  for (int l = 0; l < n_layers; ++l) {
    if ((rc = check_weights(s, &layers[l]))) return rc;
    memset(&h[l], 0, sizeof(StackLayer));
    h[l].w = layers[l];
    h[l].norm_w = norm_w ? norm_w[l] : nullptr;
    if (h[l].norm_w && ((uintptr_t)h[l].norm_w & 15)) return AINFER_ERR_ARG;
  }
  hipStream_t st = (hipStream_t)stream;
  HIP_TRY(hipMemcpyAsync(table, h.data(), h.size() * sizeof(StackLayer), hipMemcpyHostToDevice,
                         st));
  HIP_TRY(hipStreamSynchronize(st));
  // the host keeps its own copy for the replayed form, which launches the
  // layers' kernels from the host
  std::lock_guard<std::mutex> lock(g_tables_mu);
  g_tables[table] = std::move(h);
  return AINFER_OK;
}

size_t ainfer_moe_stack_workspace_bytes(const ainfer_moe_shape *s, int32_t max_tokens,
                                        int32_t n_layers) {
  if (ainfer_moe_validate(s) != AINFER_OK) return 0;
  if (max_tokens < 1 || max_tokens > AINFER_MOE_MAX_TOKENS || n_layers < 1) return 0;
  size_t need = layout_of(*s, chunk_of(max_tokens)).total;  // the replayed form
  StackGeom g;
  if (max_tokens <= DECODE_NORM_MAX_T && stack_geometry(*s, max_tokens, &g)) {
    const size_t p = layout_of(*s, 1).total + (size_t)n_layers * stack_layer_bytes(*s, max_tokens, nullptr);
    if (p > need) need = p;  // the persistent form's per-layer regions
  }
  return need;
}

namespace {
int check_stack_args(const ainfer_moe_shape *s, const void *table, int32_t n_layers,
                     int32_t norm_mode, float eps, const void *resid_in, const void *resid_out,
                     int32_t T, int max_t) {
  int rc = ainfer_moe_validate(s);
  if (rc) return rc;
  if (T < 0 || T > max_t) return AINFER_ERR_TOKENS;
  if (n_layers < 0) return AINFER_ERR_ARG;
  if (norm_mode != AINFER_NORM_PLAIN && norm_mode != AINFER_NORM_ONE_PLUS) return AINFER_ERR_ARG;
  if (!(eps >= 0.0f)) return AINFER_ERR_ARG;
  if (T == 0 || n_layers == 0) return AINFER_OK;
  if (!table || !resid_in || !resid_out) return AINFER_ERR_NULL;
  if (((uintptr_t)table) & 15 || ((uintptr_t)resid_in) & 15 || ((uintptr_t)resid_out) & 15)
    return AINFER_ERR_ARG;
  return AINFER_OK;
}

// The replayed stack on one chunk of at most CHUNK tokens.  Where the block's
// routing kernel normalizes x itself (decode, T <= 4) and in W4A8, the layers
// are the per-block entry's calls as they are.  Elsewhere the first layer's
// RMSNorm is a launch of its own and every later one is computed by the
// previous layer's combine, from the rows it writes (launch_combine_norm),
// into the workspace's h; the values are those the block entry computes.
int do_stack(const ainfer_moe_shape *s, const std::vector<StackLayer> &ly, int n_layers,
             int norm_mode, float eps, const void *resid_in, void *resid_out, int T, void *ws,
             hipStream_t st) {
  DecodeGeom dg;
  const bool folded = T <= DECODE_NORM_MAX_T && s->n_experts <= 1024 &&
                      (s->precision == AINFER_PRECISION_W4A8 || decode_geometry(*s, &dg));
  if (folded || s->precision == AINFER_PRECISION_W4A8) {
    for (int l = 0; l < n_layers; ++l) {
      int rc = do_block(s, &ly[l].w, ly[l].norm_w, norm_mode, eps, l ? resid_out : resid_in,
                        resid_out, T, ws, st);
      if (rc) return rc;
    }
    return AINFER_OK;
  }
  const Layout L = layout_of(*s, T);
  void *h = at<void>(ws, L.h);
  for (int l = 0; l < n_layers; ++l) {
    ProfCall pc(st);
    pc.start();
    if (l == 0)
      HIP_TRY(launch_rmsnorm(resid_in, ly[0].norm_w, norm_mode, eps, h, T, s->hidden, st));
    pc.end(0);
    NormIn nx;
    nx.w = l + 1 < n_layers ? (const uint16_t *)ly[l + 1].norm_w : nullptr;
    nx.mode = norm_mode;
    nx.eps = eps;
    nx.on = 1;
    int rc = do_forward(s, &ly[l].w, h, l ? resid_out : resid_in, resid_out, T, ws, st, &pc,
                        nullptr, l + 1 < n_layers ? &nx : nullptr, h);
    if (rc) return rc;
  }
  return AINFER_OK;
}
}  // namespace

int ainfer_moe_stack_forward(const ainfer_moe_shape *s, const void *table, int32_t n_layers,
                             int32_t norm_mode, float eps, const void *resid_in,
                             void *resid_out, int32_t T, void *ws, size_t ws_bytes,
                             void *stream) {
  int rc = check_stack_args(s, table, n_layers, norm_mode, eps, resid_in, resid_out, T,
                            AINFER_MOE_MAX_TOKENS);
  if (rc || T == 0 || n_layers == 0) return rc;
  if ((rc = check_ws(s, chunk_of(T), ws, ws_bytes))) return rc;
  std::vector<StackLayer> ly;
  {
    std::lock_guard<std::mutex> lock(g_tables_mu);
    auto it = g_tables.find(table);
    if (it == g_tables.end() || (int)it->second.size() < n_layers) return AINFER_ERR_ARG;
    ly.assign(it->second.begin(), it->second.begin() + n_layers);
  }
  // tokens are independent through the whole stack: each chunk runs all layers
  const size_t row = (size_t)s->hidden * 2;
  for (int t0 = 0; t0 < T; t0 += CHUNK)
    if ((rc = do_stack(s, ly, n_layers, norm_mode, eps, (const char *)resid_in + t0 * row,
                       (char *)resid_out + t0 * row, chunk_of(T - t0), ws, (hipStream_t)stream)))
      return rc;
  return strict_finish(AINFER_OK, ws, stream);
}

int ainfer_moe_stack_forward_persistent(const ainfer_moe_shape *s, const void *table,
                                        int32_t n_layers, int32_t norm_mode, float eps,
                                        const void *resid_in, void *resid_out, int32_t T,
                                        void *ws, size_t ws_bytes, void *stream) {
  int rc = check_stack_args(s, table, n_layers, norm_mode, eps, resid_in, resid_out, T,
                            DECODE_NORM_MAX_T);
  if (rc || T == 0 || n_layers == 0) return rc;
  StackGeom g;
  if (!stack_geometry(*s, T, &g)) return AINFER_ERR_SHAPE;
  if (!ws) return AINFER_ERR_NULL;
  if (((uintptr_t)ws) & 255) return AINFER_ERR_WORKSPACE;
  const Layout L = layout_of(*s, 1);
  if (ws_bytes < L.total + (size_t)n_layers * stack_layer_bytes(*s, T, nullptr))
    return AINFER_ERR_WORKSPACE;
  StackWs w;
  w.flags = at<int32_t>(ws, L.stack_flags);
  w.cap = (int)L.stack_cap;
  w.layers = at<uint8_t>(ws, L.total);
  w.err = at<int32_t>(ws, L.sync) + SY_ERR;
  HIP_TRY(launch_decode_stack(s->scale_dtype, *s, g, (const StackLayer *)table, n_layers,
                              resid_in, resid_out, T, norm_mode, eps, w, (hipStream_t)stream));
  return strict_finish(AINFER_OK, ws, stream);
}

int ainfer_moe_route(const ainfer_moe_shape *s, const ainfer_moe_weights *w, const void *x,
                     int32_t T, int32_t *topk_idx, float *topk_w, float *shared_gate,
                     float *logits, void *ws, size_t ws_bytes, void *stream) {
  int rc = ainfer_moe_validate(s);
  if (rc) return rc;
  if (T < 0 || T > AINFER_MOE_MAX_TOKENS) return AINFER_ERR_TOKENS;
  if (!w || !w->router_w) return AINFER_ERR_NULL;
  if (T == 0) return AINFER_OK;
  if (!x || !topk_idx || !topk_w || !shared_gate) return AINFER_ERR_NULL;
  if ((rc = check_ws(s, chunk_of(T), ws, ws_bytes))) return rc;
  const int H = s->hidden, E = s->n_experts, k = s->top_k;
  for (int t0 = 0; t0 < T; t0 += CHUNK)
    if ((rc = do_route(s, w, (const char *)x + (size_t)t0 * H * 2, chunk_of(T - t0),
                       topk_idx + (size_t)t0 * k, topk_w + (size_t)t0 * k, shared_gate + t0,
                       logits ? logits + (size_t)t0 * E : nullptr, ws, (hipStream_t)stream)))
      return rc;
  return AINFER_OK;
}

int ainfer_moe_experts(const ainfer_moe_shape *s, const ainfer_moe_weights *w, const void *x,
                       const int32_t *topk_idx, int32_t T, void *o, void *ws, size_t ws_bytes,
                       void *stream) {
  int rc = ainfer_moe_validate(s);
  if (rc) return rc;
  if (s->precision != AINFER_PRECISION_W4A16) return AINFER_ERR_ARG;
  if (T < 0 || T > AINFER_MOE_CHUNK_TOKENS) return AINFER_ERR_TOKENS;
  if ((rc = check_weights(s, w))) return rc;
  if (T == 0) return AINFER_OK;
  if (!x || !topk_idx || !o) return AINFER_ERR_NULL;
  if ((uintptr_t)x % 16 || (uintptr_t)o % 16) return AINFER_ERR_ARG;
  if ((rc = check_ws(s, T, ws, ws_bytes))) return rc;
  hipStream_t st = (hipStream_t)stream;
  const Layout L = layout_of(*s, T);
  const int H = s->hidden, k = s->top_k, has_shared = s->shared_inter > 0;
  const bool gemm = T >= GEMM_MIN_T;
  DispatchOut d = dispatch_out(s, L, ws, T);
  d.mt = gemm ? GEMM_MT : DEC_MT;
  if (gemm) d.small_max = GEMM_SMALL_MAX;
  ProfCall pc(st);
  pc.start();
  HIP_TRY(launch_xperm(x, at<uint16_t>(ws, L.xperm), gemm ? at<float>(ws, L.xsum) : nullptr, T,
                       H, st));
  HIP_TRY(launch_dispatch(topk_idx, T, k, s->n_experts, d.mt, has_shared,
                          at<int32_t>(ws, L.chunk_counts), at<int32_t>(ws, L.rank), d, st));
  pc.end(3);
  HIP_TRY_RC(run_experts(s, w, L, ws, d, T, gemm, st, &pc));
  HIP_TRY(launch_gather_rows(at<uint16_t>(ws, L.o), d.inv, o, T, k, H, has_shared, st));
  return AINFER_OK;
}

int ainfer_moe_combine(const ainfer_moe_shape *s, const void *o, const float *topk_w,
                       const float *shared_gate, const void *resid, void *y, int32_t T,
                       void *stream) {
  int rc = ainfer_moe_validate(s);
  if (rc) return rc;
  if (T < 0 || T > AINFER_MOE_MAX_TOKENS) return AINFER_ERR_TOKENS;
  if (T == 0) return AINFER_OK;
  const int has_shared = s->shared_inter > 0;
  if (!o || !topk_w || !y || (has_shared && !shared_gate)) return AINFER_ERR_NULL;
  if ((uintptr_t)o % 16 || (uintptr_t)y % 16 || (resid && (uintptr_t)resid % 16))
    return AINFER_ERR_ARG;
  HIP_TRY(launch_combine((const uint16_t *)o, nullptr, topk_w, shared_gate, has_shared, resid, y,
                         T, s->top_k, s->hidden, nullptr, (hipStream_t)stream));
  return AINFER_OK;
}

int ainfer_moe_dispatch(const ainfer_moe_shape *s, const int32_t *topk_idx, int32_t T,
                        int32_t *counts, int32_t *offsets, int32_t *perm, int32_t *inv_perm,
                        void *ws, size_t ws_bytes, void *stream) {
  int rc = ainfer_moe_validate(s);
  if (rc) return rc;
  if (T < 0 || T > AINFER_MOE_CHUNK_TOKENS) return AINFER_ERR_TOKENS;
  if (!counts || !offsets) return AINFER_ERR_NULL;
  if (T > 0 && (!topk_idx || !perm)) return AINFER_ERR_NULL;
  if ((rc = check_ws(s, T, ws, ws_bytes))) return rc;
  const Layout L = layout_of(*s, T);
  DispatchOut d;
  memset(&d, 0, sizeof d);
  d.counts = counts;
  d.offsets = offsets;
  d.perm = perm;
  d.inv = inv_perm;
  HIP_TRY(launch_dispatch(topk_idx, T, s->top_k, s->n_experts, SMALL_MT, s->shared_inter > 0,
                          at<int32_t>(ws, L.chunk_counts), at<int32_t>(ws, L.rank), d,
                          (hipStream_t)stream));
  return AINFER_OK;
}

int ainfer_moe_rmsnorm(const void *x, const void *w, int32_t norm_mode, float eps, void *y,
                       int32_t T, int32_t H, void *stream) {
  if (T < 0 || T > AINFER_MOE_MAX_TOKENS) return AINFER_ERR_TOKENS;
  if (H <= 0 || H % 8) return AINFER_ERR_SHAPE;
  if (norm_mode != AINFER_NORM_PLAIN && norm_mode != AINFER_NORM_ONE_PLUS) return AINFER_ERR_ARG;
  if (T == 0) return AINFER_OK;
  if (!x || !y) return AINFER_ERR_NULL;
  HIP_TRY(launch_rmsnorm(x, w, norm_mode, eps, y, T, H, (hipStream_t)stream));
  return AINFER_OK;
}

int ainfer_moe_act_quant_i8(const void *x, int32_t x_dtype, int32_t T, int32_t K, int8_t *q,
                            float *sq, void *stream) {
  if (T < 0 || T > AINFER_MOE_MAX_TOKENS) return AINFER_ERR_TOKENS;
  if (K <= 0 || K % 128) return AINFER_ERR_SHAPE;
  if (x_dtype != AINFER_ACT_F32 && x_dtype != AINFER_ACT_BF16) return AINFER_ERR_ARG;
  if (T == 0) return AINFER_OK;
  if (!x || !q || !sq) return AINFER_ERR_NULL;
  if ((uintptr_t)x % 8 || (uintptr_t)q % 2 || (uintptr_t)sq % 4) return AINFER_ERR_ARG;
  HIP_TRY(launch_act_quant_i8(x, x_dtype, T, K, q, sq, (hipStream_t)stream));
  return AINFER_OK;
}

int ainfer_moe_int4_gemv_i8(const uint8_t *packed, const void *scales, int32_t scale_dtype,
                            const int8_t *q, const float *sq, int32_t M, int32_t K, int32_t T,
                            float *y, void *stream) {
  if (T < 0 || T > AINFER_MOE_MAX_TOKENS) return AINFER_ERR_TOKENS;
  if (M <= 0 || K <= 0 || K % 128) return AINFER_ERR_SHAPE;
  if (scale_dtype != AINFER_SCALE_BF16 && scale_dtype != AINFER_SCALE_FP16) return AINFER_ERR_ARG;
  if (T == 0) return AINFER_OK;
  if (!packed || !scales || !q || !sq || !y) return AINFER_ERR_NULL;
  if ((uintptr_t)packed % 16 || (uintptr_t)q % 16 || (uintptr_t)scales % 2 ||
      (uintptr_t)sq % 4 || (uintptr_t)y % 4)
    return AINFER_ERR_ARG;
  HIP_TRY(launch_int4_gemv_i8(packed, scales, scale_dtype, q, sq, M, K, T, y, (hipStream_t)stream));
  return AINFER_OK;
}

int ainfer_moe_profile_enable(int32_t enable) {
  if (enable && !g_prof.created) {
    for (int i = 0; i < PROF_SLOTS; ++i)
      for (int j = 0; j <= NSTAGE; ++j) {
        if (hipEventCreate(&g_prof.ev[i][j]) != hipSuccess) return AINFER_ERR_HIP;
        g_prof.used[i][j] = false;
      }
    for (int i = 0; i < PROF_SLOTS; ++i) {
      for (int j = 0; j < 2; ++j)
        if (hipEventCreate(&g_prof.kev[i][j]) != hipSuccess) return AINFER_ERR_HIP;
      g_prof.kused[i] = false;
    }
    g_prof.created = true;
  }
  if (enable) {
    for (int i = 0; i < NSTAGE; ++i) g_prof.sum_us[i] = 0.0, g_prof.cnt[i] = 0;
    g_prof.calls = 0;
    g_prof.slot = 0;
    g_prof.ksum_us = 0.0;
    g_prof.kcnt = 0;
    if (g_prof.created)
      for (int i = 0; i < PROF_SLOTS; ++i) {
        for (int j = 0; j <= NSTAGE; ++j) g_prof.used[i][j] = false;
        g_prof.kused[i] = false;
      }
  }
  g_prof.on = enable != 0;
  return AINFER_OK;
}

int ainfer_moe_profile_read(float *stage_us, int32_t n_stages, int32_t *n_calls) {
  if (!stage_us && n_stages > 0) return AINFER_ERR_NULL;
  if (g_prof.created)
    for (int i = 0; i < PROF_SLOTS; ++i) prof_flush_slot(i);
  for (int i = 0; i < n_stages && i < NSTAGE; ++i)
    stage_us[i] = g_prof.cnt[i] ? (float)(g_prof.sum_us[i] / g_prof.cnt[i]) : 0.0f;
  if (n_calls) *n_calls = g_prof.calls;
  return AINFER_OK;
}

int ainfer_moe_profile_kernel(float *gate_up_us, int32_t *n_launches) {
  if (!gate_up_us) return AINFER_ERR_NULL;
  if (g_prof.created)
    for (int i = 0; i < PROF_SLOTS; ++i) prof_flush_slot(i);
  *gate_up_us = g_prof.kcnt ? (float)(g_prof.ksum_us / g_prof.kcnt) : 0.0f;
  if (n_launches) *n_launches = g_prof.kcnt;
  return AINFER_OK;
}

int ainfer_moe_debug_spin_limit(int32_t polls) {
  if (polls < 0) return AINFER_ERR_ARG;
  g_spin_max = polls;
  return AINFER_OK;
}

int ainfer_moe_fill(int32_t kind, uint64_t seed, float std_, size_t n, void *out,
                    void *stream) {
  if (kind < AINFER_FILL_BYTES || kind > AINFER_FILL_BF16_ABSNORMAL) return AINFER_ERR_ARG;
  if (n == 0) return AINFER_OK;
  if (!out) return AINFER_ERR_NULL;
  HIP_TRY(launch_fill(kind, seed, std_, n, out, (hipStream_t)stream));
  return AINFER_OK;
}

}  // extern "C"
