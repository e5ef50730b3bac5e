/*
 * moe_oracle.h - CPU oracle for the INT4 MoE layer.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker the parity tests,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg compare the HIP
 * path against.  The product (ainfer_amd/, libainfer_moe.so) never links,
 * loads or calls it.
 *
 * Every function restates the reference's arithmetic (file:line cited at
 * each definition in moe_oracle.c) or, for pieces the reference does not
 * have (router softmax/top-k/renorm, shared sigmoid gate, dispatch,
 * combine), the layer semantics documented in include/ainfer_moe.h.
 *
 * Parity pinning (what checks each function, in tests/test_oracle.py):
 *   mo_dequant_int4     hand-derived golden bytes; round trip with
 *                       mo_quantize_int4 (binfer.py:76-102 restatement)
 *   mo_quantize_int4    hand-derived golden (exact halves, clip, zero group)
 *   mo_silu_mul         reference/operators_t14.npz g,u,silu_gate_out
 *   mo_rmsnorm_f32      reference/operators_t14.npz rmsnorm_in/w/out (PLAIN)
 *   mo_router_dot       exact fp64 dot within fp32 error bound; brute-force
 *                       permutation invariance of the selected set
 *   mo_topk             brute-force sort on small inputs; tie fixtures of
 *                       tools/sample/sample.cpp:128-160; the reference
 *                       sampler (tools/sample/sampler.h) built into
 *                       oracle/_ref when /root/reference is present
 *   mo_dispatch         invariants (permutation, expert-contiguous, stable,
 *                       counts sum to T*k) + brute force on tiny inputs
 *   mo_forward          dense fp64 recomputation on tiny shapes (all
 *                       experts evaluated, combine by explicit weights)
 *   mo_fill             closed-form moments; byte-level golden values
 *   mo_act_quant_i8     numpy float32 restatement; hand-derived golden
 *                       (zero group -> scale 1, exact halves away from 0,
 *                       the group max -> +-127)
 *   mo_int4_gemv_i8     group dots against an int64 numpy matmul of the
 *                       unpacked nibbles; the float32 group-order rescale
 *                       restated in numpy (bit-exact); fp64 dequantised dot
 *                       within the fp32 rounding bound
 */
#ifndef MOE_ORACLE_H
#define MOE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#include "../include/ainfer_moe.h"

#ifdef __cplusplus
extern "C" {
#endif

/* bit conversions */
float mo_bf16_to_f32(uint16_t b);
uint16_t mo_f32_to_bf16(float f);
float mo_fp16_to_f32(uint16_t h);
uint16_t mo_f32_to_fp16(float f);

/* synthetic data, same definition as ainfer_moe_fill */
uint64_t mo_rnd(uint64_t seed, uint64_t i);
void mo_fill(int kind, uint64_t seed, float std_, size_t n, void *out);

/* INT4 g128 */
void mo_dequant_int4(const uint8_t *packed, const void *scales, int scale_dtype,
                     int rows, int K, float *out);
void mo_quantize_int4(const float *w, int rows, int K, uint8_t *packed,
                      uint16_t *scales_bf16);

/* W4A8 GEMV numerics */
void mo_act_quant_i8(const float *x, const uint16_t *x_bf16, int T, int K, int8_t *q,
                     float *sq);
void mo_int4_gemv_i8(const uint8_t *packed, const void *scales, int scale_dtype,
                     const int8_t *q, const float *sq, int M, int K, int T, float *y);
void mo_ref_gemv_inputs(int M, int K, int n_vec, uint8_t *packed, uint16_t *scales_bf16,
                        float *x);

/* pointwise */
void mo_silu_mul(const double *g, const double *u, double *out, int n);
/* fp64 sum of squares in the reference RMSNormW order (tree at N = 5120,
 * sequential otherwise) */
double mo_rms_sumsq(const float *x, int H);
void mo_rmsnorm_f32(const float *x, const float *w, int mode, float eps,
                    float *y, int T, int H);
void mo_rmsnorm_bf16(const uint16_t *x, const uint16_t *w, int mode, float eps,
                     uint16_t *y, int T, int H);

/* router */
float mo_router_dot(const uint16_t *x, const uint16_t *w, int H);
void mo_router(const ainfer_moe_shape *s, const ainfer_moe_weights *wts,
               const uint16_t *x, int T, float *logits, float *sg_logit,
               int nthreads);
void mo_topk(const float *logits, int T, int E, int k, int32_t *idx,
             float *w);
void mo_route(const ainfer_moe_shape *s, const ainfer_moe_weights *wts,
              const uint16_t *x, int T, int32_t *idx, float *w, float *sg,
              float *logits, int nthreads);
void mo_dispatch(const int32_t *idx, int T, int k, int E, int32_t *counts,
                 int32_t *offsets, int32_t *perm, int32_t *inv);

/* full layer: y_f32[T][H] fp32 and y_bf16 (either may be NULL) */
int mo_forward(const ainfer_moe_shape *s, const ainfer_moe_weights *wts,
               const uint16_t *x, int T, float *y_f32, uint16_t *y_bf16,
               int nthreads);
/* one block: h = rmsnorm(resid_in); resid_out = bf16(resid_in + moe(h)) */
int mo_block_forward(const ainfer_moe_shape *s, const ainfer_moe_weights *wts,
                     const uint16_t *norm_w, int norm_mode, float eps,
                     const uint16_t *resid_in, uint16_t *resid_out, int T,
                     int nthreads);
/* dense reference for tiny shapes: every expert evaluated, fp64 */
int mo_forward_dense(const ainfer_moe_shape *s, const ainfer_moe_weights *wts,
                     const uint16_t *x, int T, const int32_t *idx,
                     const float *w, const float *sg, double *y);

/* The layer in W4A8 (per-group int8 activations, Int4Gemv products, fp32
 * SiluMul and combine): y_f32 [T][H]. */
int mo_forward_w4a8(const ainfer_moe_shape *s, const ainfer_moe_weights *wts, const uint16_t *x,
                    int T, float *y_f32, int nthreads);

#ifdef __cplusplus
}
#endif
#endif
