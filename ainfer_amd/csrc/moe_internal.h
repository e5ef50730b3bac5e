// moe_internal.h - host-side launchers shared between the kernel files and
// the C-ABI implementation (moe_api.hip).  Not part of the public ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

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
  float *o;                   // MODE 1 out: [Tk + T][H] fp32
  const int32_t *perm;        // dispatch permutation
  const int32_t *offsets;     // [E+1]
  const int2 *tiles;          // (expert, first row) list
  const int32_t *n_tiles;
  int T, k, E, H, I, Is;
};

hipError_t launch_fill(int kind, uint64_t seed, float std_, size_t n, void *out,
                       hipStream_t s);
hipError_t launch_rmsnorm(const void *x, const void *w, int mode, float eps, void *y,
                          int T, int H, hipStream_t s);
hipError_t launch_router(const void *x, const void *rw, const float *bias, const void *gw,
                         float *logits, float *sg_logit, int T, int H, int E,
                         hipStream_t s);
hipError_t launch_topk(const float *logits, const float *sg_logit, int has_gate,
                       const void *x, int32_t *idx, float *w, float *sg, void *xperm, int T,
                       int E, int k, int H, hipStream_t s);
hipError_t launch_dispatch(const int32_t *idx, int T, int k, int E, int mt, int has_shared,
                           int32_t *chunk_counts, int32_t *rank, int32_t *counts,
                           int32_t *offsets, int32_t *perm, int32_t *inv, int2 *tiles,
                           int32_t *n_tiles, hipStream_t s);
hipError_t launch_combine(const float *o, const int32_t *inv, const float *w, const float *sg,
                          int has_shared, const void *resid, void *y, int T, int k, int H,
                          hipStream_t s);
// mode 0: gate/up + SiLU-mul; mode 1: down.  max_tiles bounds the tile list.
hipError_t launch_expert_small(int mode, int scale_dtype, const ExpertArgs &a, int max_tiles,
                               hipStream_t s);

// tile height of the small-M expert kernels
constexpr int SMALL_MT = 16;
