/*
 * moe_oracle.c - CPU oracle for the INT4 MoE layer (test infrastructure).
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * this library, and only as the checker (or as the timed CPU baseline).  The
 * product never links it.  Build: oracle/Makefile (gcc, -ffp-contract=off so
 * every fp32 operation rounds exactly where this source says it does).
 *
 * Which reference lines each function restates is given at each function.
 * Functions with no reference counterpart (the reference is a dense model,
 * see tools/decode/decode_l0.cpp:663-674) follow the semantics documented in
 * include/ainfer_moe.h and are pinned by brute force and invariants in
 * tests/test_oracle.py.
 */
#define _GNU_SOURCE
#include "moe_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* bit conversions                                                           */
/* ------------------------------------------------------------------------ */
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* bf16 <-> f32: tools/binfer.py:68-73 (f32_to_bf16_bits: round half to even
 * on the upper 16 bits; bf16_bits_to_f32: shift left 16). */
float mo_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }
uint16_t mo_f32_to_bf16(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

/* IEEE binary16, written out from the format definition. */
float mo_fp16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
  if (e == 0x1F) return u2f(sign | 0x7F800000u | (m << 13));
  if (e == 0) {
    float v = (float)m * 5.9604644775390625e-08f; /* m * 2^-24, exact */
    return sign ? -v : v;
  }
  return u2f(sign | ((e + 112u) << 23) | (m << 13));
}
uint16_t mo_f32_to_fp16(float f) {
  uint32_t x = f2u(f);
  uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7FFFFFFFu;
  if (ax >= 0x7F800000u) return (uint16_t)(sign | (ax > 0x7F800000u ? 0x7E00u : 0x7C00u));
  if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* >= 65520 -> inf */
  if (ax < 0x38800000u) {                                    /* below 2^-14    */
    uint32_t e = ax >> 23;
    if (e < 102) return (uint16_t)sign;                      /* < 2^-25        */
    uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
    uint32_t shift = 126u - e;                               /* 14..24         */
    uint32_t r = m >> shift, rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (r & 1u))) r++;
    return (uint16_t)(sign | r);
  }
  uint32_t r = ax - 0x38000000u; /* rebias 127 -> 15 */
  uint32_t out = r >> 13, rem = r & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (out & 1u))) out++;
  return (uint16_t)(sign | out);
}

static inline float scale_at(const void *scales, int dtype, size_t i) {
  uint16_t b = ((const uint16_t *)scales)[i];
  return dtype == AINFER_SCALE_FP16 ? mo_fp16_to_f32(b) : mo_bf16_to_f32(b);
}

/* ------------------------------------------------------------------------ */
/* synthetic data: counter-based splitmix64                                  */
/* The reference's harnesses use a 64-bit LCG (tools/gemv/gemv.cpp:506-515);  */
/* a counter-based generator is used here so a GPU fill can reproduce any    */
/* element independently.  Element i of stream `seed` is                     */
/* mix(seed + (i+1) * golden), i.e. the i-th output of splitmix64.           */
/* ------------------------------------------------------------------------ */
uint64_t mo_rnd(uint64_t seed, uint64_t i) {
  uint64_t z = seed + (i + 1u) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

/* standardised Irwin-Hall(8) over the 8 bytes of one 64-bit draw:
 * mean 8*127.5 = 1020, variance 8*(256^2-1)/12 = 43690 */
static inline float std_normal(uint64_t r) {
  int s = 0;
  for (int b = 0; b < 8; ++b) s += (int)((r >> (8 * b)) & 0xFFu);
  return (float)(s - 1020) * 0x1.39897ep-8f; /* 1/sqrt(43690) in fp32 */
}

void mo_fill(int kind, uint64_t seed, float std_, size_t n, void *out) {
  if (kind == AINFER_FILL_BYTES) {
    uint8_t *o = (uint8_t *)out;
    for (size_t i = 0; i < n; ++i)
      o[i] = (uint8_t)(mo_rnd(seed, i >> 3) >> (8 * (i & 7)));
    return;
  }
  uint16_t *o = (uint16_t *)out;
  for (size_t i = 0; i < n; ++i) {
    float v = std_normal(mo_rnd(seed, i)) * std_;
    switch (kind) {
    case AINFER_FILL_BF16_NORMAL: o[i] = mo_f32_to_bf16(v); break;
    case AINFER_FILL_FP16_ABSNORMAL: o[i] = mo_f32_to_fp16(fabsf(v)); break;
    case AINFER_FILL_BF16_ABSNORMAL: o[i] = mo_f32_to_bf16(fabsf(v)); break;
    default: o[i] = 0;
    }
  }
}

/* ------------------------------------------------------------------------ */
/* INT4 sym g128                                                             */
/* ------------------------------------------------------------------------ */
/* dequantize_int4_sym, tools/binfer.py:94-102: low nibble = even index,
 * nibble >= 8 -> nibble - 16, times the group's scale.  Same unpacking as
 * the host reference tools/gemv/gemv.cpp:479-501. */
void mo_dequant_int4(const uint8_t *packed, const void *scales, int scale_dtype,
                     int rows, int K, float *out) {
  int G = K / 128;
  for (int r = 0; r < rows; ++r)
    for (int k = 0; k < K; ++k) {
      size_t idx = (size_t)r * K + k;
      uint8_t b = packed[idx >> 1];
      int nib = (k & 1) ? (b >> 4) : (b & 0xF);
      if (nib >= 8) nib -= 16;
      out[idx] = (float)nib * scale_at(scales, scale_dtype, (size_t)r * G + k / 128);
    }
}

/* quantize_int4_sym, tools/binfer.py:76-91 (and pack_int4,
 * tools/gemv/gemv.cpp:46-71): scale = amax/7 (amax 0 -> 1), q =
 * clip(rint(w/scale), -8, 7) with rint = round half to even, bf16 scales.
 * The binfer.py form divides by the fp32 scale before the bf16 rounding. */
void mo_quantize_int4(const float *w, int rows, int K, uint8_t *packed,
                      uint16_t *scales_bf16) {
  int G = K / 128;
  for (int r = 0; r < rows; ++r)
    for (int g = 0; g < G; ++g) {
      const float *src = w + (size_t)r * K + (size_t)g * 128;
      float amax = 0.f;
      for (int j = 0; j < 128; ++j) amax = fmaxf(amax, fabsf(src[j]));
      float sc = amax == 0.f ? 1.0f : amax / 7.0f;
      scales_bf16[(size_t)r * G + g] = mo_f32_to_bf16(sc);
      for (int j = 0; j < 128; ++j) {
        float q = nearbyintf(src[j] / sc);
        int qi = q < -8.f ? -8 : (q > 7.f ? 7 : (int)q);
        size_t idx = (size_t)r * K + (size_t)g * 128 + j;
        if (idx & 1)
          packed[idx >> 1] |= (uint8_t)((qi & 0xF) << 4);
        else
          packed[idx >> 1] = (uint8_t)(qi & 0xF);
      }
    }
}

/* ------------------------------------------------------------------------ */
/* pointwise                                                                 */
/* ------------------------------------------------------------------------ */
/* W4A8: the reference's production GEMV numerics                           */
/* ------------------------------------------------------------------------ */
/* ScalesMax + Quantize, tools/cmdlist/kernels.cpp:551-579 (host form
 * tools/cmdlist/gemv_replay.cpp:193-204): per group of 128, m = running max
 * of |x| (a > m ? a : m from 0), sq = m / 127 (0 -> 1), q = (int)(v + 0.5)
 * for v = x/sq >= 0 else (int)(v - 0.5), clamped to [-127, 127].  x is fp32
 * (x_bf16 NULL) or bf16. */
void mo_act_quant_i8(const float *x, const uint16_t *x_bf16, int T, int K, int8_t *q,
                     float *sq) {
  int G = K / 128;
  for (int t = 0; t < T; ++t)
    for (int g = 0; g < G; ++g) {
      size_t b = (size_t)t * K + (size_t)g * 128;
      float v[128];
      for (int j = 0; j < 128; ++j) v[j] = x ? x[b + j] : mo_bf16_to_f32(x_bf16[b + j]);
      float m = 0.f;
      for (int j = 0; j < 128; ++j) {
        float a = fabsf(v[j]);
        m = a > m ? a : m;
      }
      float s = m / 127.0f;
      if (s == 0.f) s = 1.0f;
      sq[(size_t)t * G + g] = s;
      for (int j = 0; j < 128; ++j) {
        float r = v[j] / s;
        int qi = (int)(r >= 0 ? r + 0.5f : r - 0.5f);
        q[b + j] = (int8_t)(qi < -127 ? -127 : (qi > 127 ? 127 : qi));
      }
    }
}

/* The reference GEMV test's own inputs, tools/cmdlist/gemv_replay.cpp:158-192
 * (the test generator, restated): one 64-bit LCG stream; weights drawn row
 * by row, group by group, quantised with scale amax/7 (0 -> 1, stored as
 * bf16, the unrounded fp32 scale used for the division) and lrint (half to
 * even) clamped to [-8, 7]; then n_vec activation vectors of K draws x 50. */
void mo_ref_gemv_inputs(int M, int K, int n_vec, uint8_t *packed, uint16_t *scales_bf16,
                        float *x) {
  uint64_t s = 0x9E3779B9ull;
  const float unit = 0.02f / 32768.0f;
#define MO_RND() (s = s * 6364136223846793005ull + 1442695040888963407ull, \
                  (float)((int)((s >> 33) & 0xFFFF) - 32768) * unit)
  int G = K / 128;
  memset(packed, 0, (size_t)M * K / 2);
  for (int m = 0; m < M; ++m)
    for (int g = 0; g < G; ++g) {
      float w[128], amax = 0.f;
      for (int j = 0; j < 128; ++j) {
        w[j] = MO_RND();
        amax = fmaxf(amax, fabsf(w[j]));
      }
      float sc = amax == 0.f ? 1.0f : amax / 7.0f;
      scales_bf16[(size_t)m * G + g] = mo_f32_to_bf16(sc);
      for (int j = 0; j < 128; ++j) {
        int q = (int)lrintf(w[j] / sc);
        q = q < -8 ? -8 : (q > 7 ? 7 : q);
        size_t idx = (size_t)m * K + (size_t)g * 128 + j;
        if (j & 1)
          packed[idx / 2] |= (uint8_t)((q & 0xF) << 4);
        else
          packed[idx / 2] = (uint8_t)(q & 0xF);
      }
    }
  for (size_t i = 0; i < (size_t)n_vec * K; ++i) x[i] = MO_RND() * 50.0f;
#undef MO_RND
}

/* Int4Gemv, tools/cmdlist/kernels.cpp:148-201 (host mirror
 * tools/cmdlist/gemv_replay.cpp:205-221): y[t][m] = sum over groups in
 * order of (float)gs * sc * sq[t][g], gs the int32 dot of the group's
 * nibbles (low nibble = even k, nibble >= 8 -> -16) and int8 activations.
 * Built with -ffp-contract=off, so each product and sum rounds to fp32. */
void mo_int4_gemv_i8(const uint8_t *packed, const void *scales, int scale_dtype,
                     const int8_t *q, const float *sq, int M, int K, int T, float *y) {
  int G = K / 128;
  for (int t = 0; t < T; ++t)
    for (int m = 0; m < M; ++m) {
      float acc = 0.f;
      for (int g = 0; g < G; ++g) {
        float sc = scale_at(scales, scale_dtype, (size_t)m * G + g);
        int gs = 0;
        for (int j = 0; j < 128; ++j) {
          size_t k = (size_t)g * 128 + j;
          uint8_t b = packed[((size_t)m * K + k) >> 1];
          int nib = (k & 1) ? (b >> 4) : (b & 0xF);
          if (nib >= 8) nib -= 16;
          gs += nib * (int)q[(size_t)t * K + k];
        }
        acc += (float)gs * sc * sq[(size_t)t * G + g];
      }
      y[(size_t)t * M + m] = acc;
    }
}

/* ------------------------------------------------------------------------ */
/* SiluMul, tools/cmdlist/kernels.cpp:29-37 (z = g/(1+exp(-g)) * u), as the
 * fp64 CPU form of tools/forward/fwd_oracle.py:307. */
void mo_silu_mul(const double *g, const double *u, double *out, int n) {
  for (int i = 0; i < n; ++i) out[i] = g[i] / (1.0 + exp(-g[i])) * u[i];
}

/* RMSNormW, tools/cmdlist/kernels.cpp:73-116: sum of squares in fp64,
 * inv = 1/sqrt(float(ss/N) + eps) in fp32, y = x*inv*(1+w) (ONE_PLUS) or
 * x*inv*w (PLAIN, the form of reference/operators_t14.npz).  The fp64 sum
 * follows the reference's order exactly: for N = 5120, 256 work-items each
 * sum j = l, l+256, ... sequentially, then a pairwise tree st = 128 .. 1
 * (kernels.cpp:98-107); for any other N one work-item sums j = 0 .. N-1 in
 * order (kernels.cpp:86-97, the same loop as the eager rmsnorm of
 * tools/decode/decode.cpp:512-529). */
static double sumsq_tree(const float *x, int H) {
  double ps[256];
  for (int l = 0; l < 256; ++l) {
    double ss = 0.0;
    for (int j = l; j < H; j += 256) ss += (double)x[j] * (double)x[j];
    ps[l] = ss;
  }
  for (int st = 128; st > 0; st >>= 1)
    for (int l = 0; l < st; ++l) ps[l] += ps[l + st];
  return ps[0];
}

static double sumsq_seq(const float *x, int H) {
  double ss = 0.0;
  for (int j = 0; j < H; ++j) ss += (double)x[j] * (double)x[j];
  return ss;
}

double mo_rms_sumsq(const float *x, int H) {
  return H == 5120 ? sumsq_tree(x, H) : sumsq_seq(x, H);
}

void mo_rmsnorm_f32(const float *x, const float *w, int mode, float eps,
                    float *y, int T, int H) {
  for (int t = 0; t < T; ++t) {
    const float *xr = x + (size_t)t * H;
    double tot = mo_rms_sumsq(xr, H);
    float inv = 1.0f / sqrtf((float)(tot / H) + eps);
    for (int j = 0; j < H; ++j) {
      float wt = w ? (mode == AINFER_NORM_ONE_PLUS ? 1.0f + w[j] : w[j])
                   : 1.0f;
      y[(size_t)t * H + j] = xr[j] * inv * wt;
    }
  }
}

void mo_rmsnorm_bf16(const uint16_t *x, const uint16_t *w, int mode, float eps,
                     uint16_t *y, int T, int H) {
  float *xf = (float *)malloc(sizeof(float) * H);
  float *wf = w ? (float *)malloc(sizeof(float) * H) : NULL;
  float *yf = (float *)malloc(sizeof(float) * H);
  if (wf)
    for (int j = 0; j < H; ++j) wf[j] = mo_bf16_to_f32(w[j]);
  for (int t = 0; t < T; ++t) {
    for (int j = 0; j < H; ++j) xf[j] = mo_bf16_to_f32(x[(size_t)t * H + j]);
    mo_rmsnorm_f32(xf, wf, mode, eps, yf, 1, H);
    for (int j = 0; j < H; ++j) y[(size_t)t * H + j] = mo_f32_to_bf16(yf[j]);
  }
  free(xf); free(wf); free(yf);
}

/* ------------------------------------------------------------------------ */
/* simple parallel-for                                                       */
/* ------------------------------------------------------------------------ */
typedef void (*range_fn)(void *ctx, long lo, long hi);
typedef struct { range_fn fn; void *ctx; long lo, hi; } pf_arg;
static void *pf_tramp(void *p) {
  pf_arg *a = (pf_arg *)p;
  a->fn(a->ctx, a->lo, a->hi);
  return NULL;
}
static void parallel_for(long n, int nthreads, range_fn fn, void *ctx) {
  if (nthreads > n) nthreads = (int)n;
  if (nthreads > 256) nthreads = 256;
  if (nthreads <= 1) { fn(ctx, 0, n); return; }
  pthread_t th[256];
  pf_arg args[256];
  char ok[256];
  long per = (n + nthreads - 1) / nthreads;
  for (int i = 0; i < nthreads; ++i) {
    long lo = i * per, hi = lo + per < n ? lo + per : n;
    args[i] = (pf_arg){fn, ctx, lo, hi > lo ? hi : lo};
    ok[i] = 0;
    if (i > 0 && lo < hi) ok[i] = pthread_create(&th[i], NULL, pf_tramp, &args[i]) == 0;
  }
  fn(ctx, args[0].lo, args[0].hi);
  for (int i = 1; i < nthreads; ++i) {
    if (ok[i]) pthread_join(th[i], NULL);
    else if (args[i].lo < args[i].hi) fn(ctx, args[i].lo, args[i].hi);
  }
}

/* ------------------------------------------------------------------------ */
/* router                                                                    */
/* ------------------------------------------------------------------------ */
/* The lane-strided chunk order (include/ainfer_moe.h): bf16 x bf16 products
 * are exact in fp32, each fmaf rounds once; lane l covers 8-element chunks
 * l, l+64, ...; the 64 partials are combined by an xor butterfly. */
float mo_router_dot(const uint16_t *x, const uint16_t *w, int H) {
  float part[64], nxt[64];
  int nch = H / 8;
  for (int l = 0; l < 64; ++l) {
    float acc = 0.0f;
    for (int c = l; c < nch; c += 64)
      for (int i = 0; i < 8; ++i)
        acc = fmaf(mo_bf16_to_f32(x[8 * c + i]), mo_bf16_to_f32(w[8 * c + i]), acc);
    part[l] = acc;
  }
  for (int m = 32; m >= 1; m >>= 1) {
    for (int l = 0; l < 64; ++l) nxt[l] = part[l] + part[l ^ m];
    memcpy(part, nxt, sizeof part);
  }
  return part[0];
}

typedef struct {
  const ainfer_moe_shape *s;
  const ainfer_moe_weights *w;
  const uint16_t *x;
  float *logits, *sg;
} router_ctx;
static void router_range(void *p, long lo, long hi) {
  router_ctx *c = (router_ctx *)p;
  int H = c->s->hidden, E = c->s->n_experts;
  for (long t = lo; t < hi; ++t) {
    const uint16_t *xr = c->x + (size_t)t * H;
    for (int e = 0; e < E; ++e) {
      float v = mo_router_dot(xr, (const uint16_t *)c->w->router_w + (size_t)e * H, H);
      if (c->w->router_bias) v = v + c->w->router_bias[e];
      c->logits[(size_t)t * E + e] = v;
    }
    if (c->sg)
      c->sg[t] = c->w->shared_gate_w
                     ? mo_router_dot(xr, (const uint16_t *)c->w->shared_gate_w, H)
                     : 0.0f;
  }
}
void mo_router(const ainfer_moe_shape *s, const ainfer_moe_weights *wts,
               const uint16_t *x, int T, float *logits, float *sg_logit,
               int nthreads) {
  router_ctx c = {s, wts, x, logits, sg_logit};
  parallel_for(T, nthreads, router_range, &c);
}

/* Top-k with the tie rule of tools/sample/sampler.h:90-98 (value descending,
 * equal values lower index first) and first-max-wins argmax
 * (tools/cmdlist/kernels.cpp:480-546): k passes of a strict-greater scan in
 * ascending index order.  Selection is on fp32 logits (softmax is monotone).
 * Weights: exp(l_j - l_max) / sum over the selected, in fp32. */
void mo_topk(const float *logits, int T, int E, int k, int32_t *idx, float *w) {
  char *taken = (char *)malloc((size_t)E);
  for (int t = 0; t < T; ++t) {
    const float *l = logits + (size_t)t * E;
    memset(taken, 0, (size_t)E);
    for (int j = 0; j < k; ++j) {
      int best = -1;
      for (int e = 0; e < E; ++e) {
        if (taken[e]) continue;
        if (best < 0 || l[e] > l[best]) best = e;
      }
      taken[best] = 1;
      idx[(size_t)t * k + j] = best;
    }
    float m = l[idx[(size_t)t * k]], sum = 0.0f;
    for (int j = 0; j < k; ++j) {
      float p = expf(l[idx[(size_t)t * k + j]] - m);
      w[(size_t)t * k + j] = p;
      sum += p;
    }
    for (int j = 0; j < k; ++j) w[(size_t)t * k + j] = w[(size_t)t * k + j] / sum;
  }
  free(taken);
}

void mo_route(const ainfer_moe_shape *s, const ainfer_moe_weights *wts,
              const uint16_t *x, int T, int32_t *idx, float *w, float *sg,
              float *logits, int nthreads) {
  int E = s->n_experts;
  float *lg = logits ? logits : (float *)malloc(sizeof(float) * (size_t)T * E);
  float *sgl = (float *)malloc(sizeof(float) * (size_t)(T > 0 ? T : 1));
  mo_router(s, wts, x, T, lg, sgl, nthreads);
  mo_topk(lg, T, E, s->top_k, idx, w);
  for (int t = 0; t < T; ++t)
    sg[t] = wts->shared_gate_w ? 1.0f / (1.0f + expf(-sgl[t])) : 1.0f;
  if (!logits) free(lg);
  free(sgl);
}

/* Dispatch: histogram, exclusive scan, stable placement by (expert, token). */
void mo_dispatch(const int32_t *idx, int T, int k, int E, int32_t *counts,
                 int32_t *offsets, int32_t *perm, int32_t *inv) {
  memset(counts, 0, sizeof(int32_t) * (size_t)E);
  for (long i = 0; i < (long)T * k; ++i) counts[idx[i]]++;
  offsets[0] = 0;
  for (int e = 0; e < E; ++e) offsets[e + 1] = offsets[e] + counts[e];
  int32_t *cur = (int32_t *)malloc(sizeof(int32_t) * (size_t)E);
  memcpy(cur, offsets, sizeof(int32_t) * (size_t)E);
  for (int t = 0; t < T; ++t)
    for (int j = 0; j < k; ++j) {
      int e = idx[(size_t)t * k + j];
      int p = cur[e]++;
      perm[p] = t * k + j;
      if (inv) inv[t * k + j] = p;
    }
  free(cur);
}

/* ------------------------------------------------------------------------ */
/* experts                                                                   */
/* ------------------------------------------------------------------------ */
/* One INT4 GEMV row in fp64: sum_g scale * sum_j q * x, the depacked
 * double-precision host reference of tools/gemv/gemv.cpp:479-501. */
static double int4_row_dot(const uint8_t *prow, const void *scales, int dtype,
                           size_t srow, int K, const double *x) {
  double acc = 0.0;
  int G = K / 128;
  for (int g = 0; g < G; ++g) {
    double sc = scale_at(scales, dtype, srow + g);
    const uint8_t *b = prow + (size_t)g * 64;
    const double *xg = x + (size_t)g * 128;
    double gs = 0.0;
    for (int j = 0; j < 64; ++j) {
      int lo = b[j] & 0xF, hi = b[j] >> 4;
      lo -= (lo & 8) << 1;
      hi -= (hi & 8) << 1;
      gs += lo * xg[2 * j] + hi * xg[2 * j + 1];
    }
    acc += sc * gs;
  }
  return acc;
}

/* expert(x) = W_down (silu(W_gate x) * (W_up x)), the MLP of
 * tools/decode/decode_l0.cpp:663-674 / tools/forward/fwd_oracle.py:302-310
 * without the activation re-quantisation (this layer is W4A16). */
static void expert_apply(const uint8_t *wg, const void *sg_, const uint8_t *wu,
                         const void *su, const uint8_t *wd, const void *sd,
                         int dtype, int H, int I, const double *x, double *tmp_g,
                         double *tmp_u, double *a, double *out) {
  for (int n = 0; n < I; ++n) {
    tmp_g[n] = int4_row_dot(wg + (size_t)n * (H / 2), sg_, dtype, (size_t)n * (H / 128), H, x);
    tmp_u[n] = int4_row_dot(wu + (size_t)n * (H / 2), su, dtype, (size_t)n * (H / 128), H, x);
  }
  mo_silu_mul(tmp_g, tmp_u, a, I);
  for (int h = 0; h < H; ++h)
    out[h] = int4_row_dot(wd + (size_t)h * (I / 2), sd, dtype, (size_t)h * (I / 128), I, a);
}

typedef struct {
  const ainfer_moe_shape *s;
  const ainfer_moe_weights *w;
  const uint16_t *x;
  const int32_t *idx;
  int t0;     /* first token of the chunk */
  double *o;  /* [pairs of chunk][H], pair = (t - t0) * (k + 1) + j, j == k shared */
} moe_ctx;

static void moe_range(void *p, long lo, long hi) {
  moe_ctx *c = (moe_ctx *)p;
  const ainfer_moe_shape *s = c->s;
  const ainfer_moe_weights *w = c->w;
  int H = s->hidden, I = s->inter, Is = s->shared_inter, k = s->top_k;
  int Im = I > Is ? I : Is, dt = s->scale_dtype;
  double *x = (double *)malloc(sizeof(double) * H);
  double *g = (double *)malloc(sizeof(double) * Im);
  double *u = (double *)malloc(sizeof(double) * Im);
  double *a = (double *)malloc(sizeof(double) * Im);
  for (long q = lo; q < hi; ++q) {
    int t = c->t0 + (int)(q / (k + 1)), j = (int)(q % (k + 1));
    double *o = c->o + (size_t)q * H;
    if (j == k && Is == 0) continue;
    for (int h = 0; h < H; ++h) x[h] = mo_bf16_to_f32(c->x[(size_t)t * H + h]);
    if (j < k) {
      int e = c->idx[(size_t)t * k + j];
      size_t pg = (size_t)e * I * (H / 2), sgo = (size_t)e * I * (H / 128);
      size_t pd = (size_t)e * H * (I / 2), sdo = (size_t)e * H * (I / 128);
      expert_apply(w->w_gate + pg, (const uint16_t *)w->s_gate + sgo, w->w_up + pg,
                   (const uint16_t *)w->s_up + sgo, w->w_down + pd,
                   (const uint16_t *)w->s_down + sdo, dt, H, I, x, g, u, a, o);
    } else {
      expert_apply(w->ws_gate, w->ss_gate, w->ws_up, w->ss_up, w->ws_down,
                   w->ss_down, dt, H, Is, x, g, u, a, o);
    }
  }
  free(x); free(g); free(u); free(a);
}

/* Combine: y_t = sum_j w_j o_{t,j} + g_s o_shared, in slot order, fp64.
 * Pairs are evaluated in parallel over token chunks of 64. */
int mo_forward(const ainfer_moe_shape *s, const ainfer_moe_weights *wts,
               const uint16_t *x, int T, float *y_f32, uint16_t *y_bf16,
               int nthreads) {
  int k = s->top_k, H = s->hidden, Is = s->shared_inter;
  if (T <= 0) return 0;
  const int CH = 64;
  int32_t *idx = (int32_t *)malloc(sizeof(int32_t) * (size_t)T * k);
  float *tw = (float *)malloc(sizeof(float) * (size_t)T * k);
  float *sg = (float *)malloc(sizeof(float) * (size_t)T);
  double *o = (double *)malloc(sizeof(double) * (size_t)CH * (k + 1) * H);
  mo_route(s, wts, x, T, idx, tw, sg, NULL, nthreads);
  for (int t0 = 0; t0 < T; t0 += CH) {
    int nt = T - t0 < CH ? T - t0 : CH;
    moe_ctx c = {s, wts, x, idx, t0, o};
    parallel_for((long)nt * (k + 1), nthreads, moe_range, &c);
    for (int tt = 0; tt < nt; ++tt) {
      int t = t0 + tt;
      for (int h = 0; h < H; ++h) {
        double acc = 0.0;
        for (int j = 0; j < k; ++j)
          acc += (double)tw[(size_t)t * k + j] * o[((size_t)tt * (k + 1) + j) * H + h];
        if (Is > 0) acc += (double)sg[t] * o[((size_t)tt * (k + 1) + k) * H + h];
        size_t i = (size_t)t * H + h;
        if (y_f32) y_f32[i] = (float)acc;
        if (y_bf16) y_bf16[i] = mo_f32_to_bf16((float)acc);
      }
    }
  }
  free(idx); free(tw); free(sg); free(o);
  return 0;
}

/* The layer in W4A8 (AINFER_PRECISION_W4A8): per (token, expert) the MLP
 * sequence of tools/decode/decode_l0.cpp:663-674 -- xq (ScalesMax +
 * Quantize, mo_act_quant_i8), Int4Gemv gate and up (mo_int4_gemv_i8),
 * SiluMul in fp32 (kernels.cpp:29-37: g / (1 + exp(-g)) * u), quantize,
 * Int4Gemv down -- then the combine in fp32: fmaf(w_j, o_j, acc) in slot
 * order, fmaf(g_s, o_shared, acc).  Routing as mo_route.  y_f32 [T][H]. */
typedef struct {
  const ainfer_moe_shape *s;
  const ainfer_moe_weights *w;
  const uint16_t *x;
  const int32_t *idx;
  const float *tw, *sg;
  float *y;
} w8_ctx;

static void w8_expert(const uint8_t *wg, const void *sg_, const uint8_t *wu, const void *su,
                      const uint8_t *wd, const void *sd, int dt, int H, int I, const int8_t *xq,
                      const float *xs, float *g, float *u, int8_t *aq, float *as, float *o) {
  mo_int4_gemv_i8(wg, sg_, dt, xq, xs, I, H, 1, g);
  mo_int4_gemv_i8(wu, su, dt, xq, xs, I, H, 1, u);
  for (int n = 0; n < I; ++n) g[n] = g[n] / (1.0f + expf(-g[n])) * u[n];
  mo_act_quant_i8(g, NULL, 1, I, aq, as);
  mo_int4_gemv_i8(wd, sd, dt, aq, as, H, I, 1, o);
}

static void w8_range(void *p, long lo, long hi) {
  w8_ctx *c = (w8_ctx *)p;
  const ainfer_moe_shape *s = c->s;
  const ainfer_moe_weights *w = c->w;
  int H = s->hidden, I = s->inter, Is = s->shared_inter, k = s->top_k, dt = s->scale_dtype;
  int Im = I > Is ? I : Is;
  int8_t *xq = (int8_t *)malloc((size_t)H);
  float *xs = (float *)malloc(sizeof(float) * (H / 128));
  float *g = (float *)malloc(sizeof(float) * Im), *u = (float *)malloc(sizeof(float) * Im);
  int8_t *aq = (int8_t *)malloc((size_t)Im);
  float *as = (float *)malloc(sizeof(float) * (Im / 128));
  float *o = (float *)malloc(sizeof(float) * (size_t)(k + 1) * H);
  for (long t = lo; t < hi; ++t) {
    mo_act_quant_i8(NULL, c->x + (size_t)t * H, 1, H, xq, xs);
    for (int j = 0; j < k; ++j) {
      int e = c->idx[(size_t)t * k + j];
      size_t pg = (size_t)e * I * (H / 2), sgo = (size_t)e * I * (H / 128);
      size_t pd = (size_t)e * H * (I / 2), sdo = (size_t)e * H * (I / 128);
      w8_expert(w->w_gate + pg, (const uint16_t *)w->s_gate + sgo, w->w_up + pg,
                (const uint16_t *)w->s_up + sgo, w->w_down + pd, (const uint16_t *)w->s_down + sdo,
                dt, H, I, xq, xs, g, u, aq, as, o + (size_t)j * H);
    }
    if (Is > 0)
      w8_expert(w->ws_gate, w->ss_gate, w->ws_up, w->ss_up, w->ws_down, w->ss_down, dt, H, Is,
                xq, xs, g, u, aq, as, o + (size_t)k * H);
    for (int h = 0; h < H; ++h) {
      float acc = 0.0f;
      for (int j = 0; j < k; ++j) acc = fmaf(c->tw[(size_t)t * k + j], o[(size_t)j * H + h], acc);
      if (Is > 0) acc = fmaf(c->sg[t], o[(size_t)k * H + h], acc);
      c->y[(size_t)t * H + h] = acc;
    }
  }
  free(xq); free(xs); free(g); free(u); free(aq); free(as); free(o);
}

int mo_forward_w4a8(const ainfer_moe_shape *s, const ainfer_moe_weights *wts, const uint16_t *x,
                    int T, float *y_f32, int nthreads) {
  int k = s->top_k;
  if (T <= 0) return 0;
  int32_t *idx = (int32_t *)malloc(sizeof(int32_t) * (size_t)T * k);
  float *tw = (float *)malloc(sizeof(float) * (size_t)T * k);
  float *sg = (float *)malloc(sizeof(float) * (size_t)T);
  mo_route(s, wts, x, T, idx, tw, sg, NULL, nthreads);
  w8_ctx c = {s, wts, x, idx, tw, sg, y_f32};
  parallel_for(T, nthreads, w8_range, &c);
  free(idx); free(tw); free(sg);
  return 0;
}

int mo_block_forward(const ainfer_moe_shape *s, const ainfer_moe_weights *wts,
                     const uint16_t *norm_w, int norm_mode, float eps,
                     const uint16_t *resid_in, uint16_t *resid_out, int T,
                     int nthreads) {
  int H = s->hidden;
  uint16_t *h = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)T * H);
  float *y = (float *)malloc(sizeof(float) * (size_t)T * H);
  mo_rmsnorm_bf16(resid_in, norm_w, norm_mode, eps, h, T, H);
  mo_forward(s, wts, h, T, y, NULL, nthreads);
  for (size_t i = 0; i < (size_t)T * H; ++i)
    resid_out[i] = mo_f32_to_bf16(mo_bf16_to_f32(resid_in[i]) + y[i]);
  free(h); free(y);
  return 0;
}

/* Dense fp64 form for tiny shapes: every expert is evaluated on every token
 * from fully dequantised matrices, and the output is the explicit weighted
 * sum with the given routing.  Shares no code with moe_range beyond the
 * fp64 SiLU, so it checks the sparse path's indexing. */
int mo_forward_dense(const ainfer_moe_shape *s, const ainfer_moe_weights *wts,
                     const uint16_t *x, int T, const int32_t *idx,
                     const float *w, const float *sg, double *y) {
  int H = s->hidden, I = s->inter, Is = s->shared_inter, E = s->n_experts,
      k = s->top_k, dt = s->scale_dtype;
  int Im = I > Is ? I : Is;
  float *Wg = (float *)malloc(sizeof(float) * (size_t)Im * H);
  float *Wu = (float *)malloc(sizeof(float) * (size_t)Im * H);
  float *Wd = (float *)malloc(sizeof(float) * (size_t)H * Im);
  double *out = (double *)malloc(sizeof(double) * (size_t)(E + 1) * T * H);
  double *gu = (double *)malloc(sizeof(double) * (size_t)Im * 2);
  for (int e = 0; e <= E; ++e) {
    int Ie = e < E ? I : Is;
    if (Ie == 0) continue;
    if (e < E) {
      mo_dequant_int4(wts->w_gate + (size_t)e * I * (H / 2),
                      (const uint16_t *)wts->s_gate + (size_t)e * I * (H / 128), dt, I, H, Wg);
      mo_dequant_int4(wts->w_up + (size_t)e * I * (H / 2),
                      (const uint16_t *)wts->s_up + (size_t)e * I * (H / 128), dt, I, H, Wu);
      mo_dequant_int4(wts->w_down + (size_t)e * H * (I / 2),
                      (const uint16_t *)wts->s_down + (size_t)e * H * (I / 128), dt, H, I, Wd);
    } else {
      mo_dequant_int4(wts->ws_gate, wts->ss_gate, dt, Is, H, Wg);
      mo_dequant_int4(wts->ws_up, wts->ss_up, dt, Is, H, Wu);
      mo_dequant_int4(wts->ws_down, wts->ss_down, dt, H, Is, Wd);
    }
    for (int t = 0; t < T; ++t) {
      for (int n = 0; n < Ie; ++n) {
        double ag = 0, au = 0;
        for (int h = 0; h < H; ++h) {
          double xv = mo_bf16_to_f32(x[(size_t)t * H + h]);
          ag += (double)Wg[(size_t)n * H + h] * xv;
          au += (double)Wu[(size_t)n * H + h] * xv;
        }
        gu[n] = ag / (1.0 + exp(-ag)) * au;
      }
      for (int h = 0; h < H; ++h) {
        double acc = 0;
        for (int n = 0; n < Ie; ++n) acc += (double)Wd[(size_t)h * Ie + n] * gu[n];
        out[((size_t)e * T + t) * H + h] = acc;
      }
    }
  }
  for (int t = 0; t < T; ++t)
    for (int h = 0; h < H; ++h) {
      double acc = 0;
      for (int j = 0; j < k; ++j)
        acc += (double)w[(size_t)t * k + j] * out[((size_t)idx[(size_t)t * k + j] * T + t) * H + h];
      if (Is > 0) acc += (double)sg[t] * out[((size_t)E * T + t) * H + h];
      y[(size_t)t * H + h] = acc;
    }
  free(Wg); free(Wu); free(Wd); free(out); free(gu);
  return 0;
}
