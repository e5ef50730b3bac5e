/*
 * ainfer_moe.h - C ABI of the MI355X (gfx950) INT4 mixture-of-experts layer.
 *
 * Plain C: POD structs, raw device pointers, sizes, an opaque stream handle
 * (a hipStream_t passed as void*, NULL = the default stream) and int status
 * codes.  No C++ or torch types cross this boundary.
 *
 * Conventions carried over from the reference runtime's operator surface
 * (tools/decode/decode_l0.cpp):
 *   - the caller owns every buffer, including the workspace; nothing is
 *     allocated inside a forward call (decode_l0.cpp:220-295 allocates all
 *     arenas and scratch once at init);
 *   - kernels receive raw device pointers into caller-owned weight arenas
 *     (decode_l0.cpp:494-504, the gemvE lambda);
 *   - all work is stream-ordered; a call returns after enqueueing
 *     (decode_l0.cpp:484-493 appends launch + barrier to a list);
 *   - errors are reported, never fatal: the reference CHECK()s and exits
 *     (decode_l0.cpp:26-34); this layer returns a negative status instead,
 *     with the text available from ainfer_moe_strerror().
 *
 * Weight format (per tensor, expert-contiguous):
 *   packed  [rows][K/2] uint8, two signed 4-bit values per byte, low nibble =
 *           even k, two's complement in [-8, 7]
 *           (tools/binfer.py:76-102, tools/gemv/gemv.cpp:46-71);
 *   scales  [rows][K/128] fp16 (or bf16, selected by scale_dtype), one per
 *           group of 128 consecutive k (docs/binfer_spec.md:79-91).
 *   dequantised weight w[n][k] = q[n][k] * scale[n][k/128].
 * Routed expert e: gate/up are [I][H] (rows = I, K = H), down is [H][I]
 * (rows = H, K = I); expert e's tensor starts at e * rows * K/2 bytes and
 * its scales at e * rows * K/128 elements.
 *
 * Layer semantics (one token t, x_t in bf16):
 *   logit_e   = dot(x_t, router_w[e]) (+ router_bias[e])     fp32
 *   top-k     = the k largest logits, equal logits ordered lower index first
 *               (the tie rule of tools/sample/sampler.h:97-98)
 *   w_j       = exp(logit_j - logit_max) / sum_{selected} exp(...)
 *               (= softmax over all E, keep top-k, renormalise)
 *   g_s       = sigmoid(dot(x_t, shared_gate_w))   (1 when no gate vector)
 *   expert_e(x) = W_down (silu(W_gate x) * (W_up x))
 *   y_t       = sum_j w_j * expert_{e_j}(x_t) + g_s * shared(x_t)
 * Router dot products use one fixed fp32 summation order (the "lane-strided
 * chunk order": 64 lanes, lane l sums 8-element chunks l, l+64, ...
 * sequentially with fma, then an xor butterfly over 32,16,8,4,2,1), so
 * logits, and therefore top-k indices, are bit-identical to the CPU oracle.
 * The dispatch permutation orders (token, slot) pairs by expert ascending,
 * then token ascending.
 */
#ifndef AINFER_MOE_H
#define AINFER_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
enum {
  AINFER_OK = 0,
  AINFER_ERR_SHAPE = -1,      /* shape fails validation                     */
  AINFER_ERR_NULL = -2,       /* a required pointer is NULL                 */
  AINFER_ERR_WORKSPACE = -3,  /* workspace too small or misaligned          */
  AINFER_ERR_TOKENS = -4,     /* T < 0 or above the supported maximum       */
  AINFER_ERR_HIP = -5,        /* a HIP runtime call failed                  */
  AINFER_ERR_ARG = -6,        /* another argument is out of range           */
  AINFER_ERR_SYNC = -7,       /* a device-side wait ran out (decode path)   */
  AINFER_ERR_SCRATCH = -8,    /* the call needs more than the static scratch
                                 of ainfer_moe_block_forward_noalloc holds    */
  AINFER_ERR_FORMAT = -9,     /* a .binfer file fails validation            */
  AINFER_ERR_IO = -10         /* a file cannot be opened or read            */
};

enum { AINFER_SCALE_BF16 = 0, AINFER_SCALE_FP16 = 1 };

/* Expert arithmetic of the layer entries.
 * W4A16: bf16 activations against dequantised INT4 weights, fp32 sums
 *   (bf16 MFMA), act and expert outputs rounded to bf16.
 * W4A8: the reference's production decode numerics (the MLP sequence of
 *   tools/decode/decode_l0.cpp:663-674): x quantised per group of 128 to int8
 *   (ScalesMax + Quantize, tools/cmdlist/kernels.cpp:551-579), gate and up
 *   as Int4Gemv (kernels.cpp:148-201: exact int32 group dots, fp32 terms
 *   float(gs) * s_w * s_x added in group order without contraction), act =
 *   SiluMul in fp32, quantised again, down as Int4Gemv, and the combine in
 *   fp32 (fma in slot order) before the bf16 output.  Each GEMV gives the
 *   reference formula's bits on the same inputs (ainfer_moe_int4_gemv_i8). */
enum { AINFER_PRECISION_W4A16 = 0, AINFER_PRECISION_W4A8 = 1 };

/* RMSNorm weight forms: reference RMSNormW uses y = x*inv*(1+w)
 * (tools/cmdlist/kernels.cpp:73-116); the operator fixture
 * (reference/operators_t14.npz rmsnorm_*) uses y = x*inv*w. */
enum { AINFER_NORM_PLAIN = 0, AINFER_NORM_ONE_PLUS = 1 };

/* Largest token count one call accepts. */
#define AINFER_MOE_MAX_TOKENS 65536
/* Calls with more tokens than this run as consecutive chunks of at most this
 * many tokens on one workspace (chunked prefill; the reference records its
 * prefill GEMMs per chunk, tools/cmdlist/chunkgemm_replay.cpp): the
 * workspace is the chunk's size (ainfer_moe_workspace_bytes stops growing
 * here) and each token is routed and computed within its chunk.  The
 * stage-level dispatch entry is not chunked (its permutation spans all T). */
#define AINFER_MOE_CHUNK_TOKENS 4096

typedef struct ainfer_moe_shape {
  int32_t hidden;       /* H, multiple of 128                               */
  int32_t n_experts;    /* E, 1..1024                                       */
  int32_t top_k;        /* k, 1..min(E, 32)                                 */
  int32_t inter;        /* I of each routed expert, multiple of 128         */
  int32_t shared_inter; /* I of the shared expert, multiple of 128; 0 = none */
  int32_t group;        /* quantisation group along K; must be 128          */
  int32_t scale_dtype;  /* AINFER_SCALE_FP16 or AINFER_SCALE_BF16           */
  int32_t precision;    /* AINFER_PRECISION_W4A16 (0) or _W4A8              */
} ainfer_moe_shape;

/* Device pointers.  Weight and router tensors must be 16-byte aligned, scale
 * tensors 8-byte aligned (AINFER_ERR_ARG otherwise). */
typedef struct ainfer_moe_weights {
  const void *router_w;      /* [E][H] bf16                                 */
  const float *router_bias;  /* [E] fp32 added to the logits, or NULL       */
  const void *shared_gate_w; /* [H] bf16 sigmoid gate of the shared expert,
                                or NULL (gate = 1)                          */
  const uint8_t *w_gate;     /* [E][I][H/2]                                 */
  const void *s_gate;        /* [E][I][H/128]                               */
  const uint8_t *w_up;       /* [E][I][H/2]                                 */
  const void *s_up;          /* [E][I][H/128]                               */
  const uint8_t *w_down;     /* [E][H][I/2]                                 */
  const void *s_down;        /* [E][H][I/128]                               */
  const uint8_t *ws_gate;    /* shared expert [Is][H/2] (unused if Is == 0)  */
  const void *ss_gate;       /* [Is][H/128]                                 */
  const uint8_t *ws_up;      /* [Is][H/2]                                   */
  const void *ss_up;         /* [Is][H/128]                                 */
  const uint8_t *ws_down;    /* [H][Is/2]                                   */
  const void *ss_down;       /* [H][Is/128]                                 */
} ainfer_moe_weights;

/* Text for a status code. */
const char *ainfer_moe_strerror(int status);

/* AINFER_OK when the shape is supported, AINFER_ERR_SHAPE otherwise. */
int ainfer_moe_validate(const ainfer_moe_shape *shape);

/* Bytes of device workspace one call with up to max_tokens tokens needs
 * (0 on an invalid shape).  The workspace must be 256-byte aligned. */
size_t ainfer_moe_workspace_bytes(const ainfer_moe_shape *shape,
                                  int32_t max_tokens);

/* Zero the workspace's synchronisation words (a few KB at its start).  Call
 * once after allocating a workspace, before its first forward call (a
 * workspace allocated zero-filled needs no call).  The decode path (T <= 16)
 * hands work between workgroups through counters there and every call leaves
 * them zero again.  Calls that use one workspace must not overlap.
 * Replaces the init-time arena set-up of decode_l0.cpp:220-295 for this
 * layer's scratch. */
int ainfer_moe_workspace_init(const ainfer_moe_shape *shape, void *workspace,
                              size_t workspace_bytes, void *stream);
/* Synchronise the stream and read the workspace's synchronisation words
 * back: AINFER_OK when they are all zero, AINFER_ERR_SYNC when a bounded
 * device-side wait ran out (its result is then not to be trusted; re-init
 * the workspace), AINFER_ERR_WORKSPACE when other words are left non-zero
 * (overlapping calls on one workspace).  A diagnostic, not for the hot loop;
 * it has no counterpart in the reference, whose waits are host fences
 * (decode_l0.cpp:484-493).
 * A wait that runs out also sets a sticky error word in the workspace: from
 * then on every forward/block_forward on that workspace writes NaN to all of
 * its output rows (the call itself still returns AINFER_OK, since it only
 * enqueues), until ainfer_moe_workspace_init clears the word. */
int ainfer_moe_workspace_check(const ainfer_moe_shape *shape, const void *workspace,
                               size_t workspace_bytes, void *stream);
/* The whole layer: y[T][H] (bf16) = MoE(x[T][H] bf16).
 * Replaces the reference MLP sub-sequence decode_l0.cpp:663-674
 * (xq -> gemvE gate -> gemvE up -> SiluMul -> xq -> gemvE down -> res) with
 * router -> dispatch -> grouped INT4 expert SwiGLU -> combine + shared. */
int ainfer_moe_forward(const ainfer_moe_shape *shape,
                       const ainfer_moe_weights *weights, const void *x,
                       void *y, int32_t T, void *workspace,
                       size_t workspace_bytes, void *stream);

/* One decoder-block MLP half with residual, as in decode_l0.cpp:663-674:
 *   h = RMSNorm(resid_in) (eps, norm_w in norm_mode, NULL = unit weight),
 *   resid_out = bf16(resid_in + MoE(h)).   resid_out may alias resid_in. */
int ainfer_moe_block_forward(const ainfer_moe_shape *shape,
                             const ainfer_moe_weights *weights,
                             const void *norm_w, int32_t norm_mode, float eps,
                             const void *resid_in, void *resid_out, int32_t T,
                             void *workspace, size_t workspace_bytes,
                             void *stream);

/* ---- decode stack: many blocks in one call ------------------------------
 * The reference records each layer's command list once at init and replays
 * the recorded lists every decode step (tools/decode/decode_l0.cpp:553-677,
 * the MLP part :663-674).  Here the init step writes a device table of the
 * layers' weights (ainfer_moe_stack_prepare, which also keeps a host copy)
 * and one call runs all of them:
 *   for l in 0..n_layers-1:  r = bf16(r + MoE_l(RMSNorm_l(r)))
 * with r = resid_in at the start and resid_out at the end (resid_out may
 * alias resid_in).  Each layer's output is bit-identical to
 * ainfer_moe_block_forward on the same input, so the stack equals n_layers
 * chained block_forward calls.
 *
 * ainfer_moe_stack_forward replays the layers' kernels from the host, any T
 * up to AINFER_MOE_MAX_TOKENS (chunks of AINFER_MOE_CHUNK_TOKENS each run
 * every layer).  Where the block entry would launch an RMSNorm of its own
 * (T > 4, W4A16), the previous layer's combine computes it from the rows it
 * writes (the residual add fused into the next norm, tools/norm/norm.cpp:
 * 30-61), so a layer is one launch shorter.  The table must come from
 * ainfer_moe_stack_prepare in this process (else AINFER_ERR_ARG; the host
 * copy, a few hundred bytes per layer, is kept until the process ends or the
 * same table address is prepared again); workspace:
 * ainfer_moe_stack_workspace_bytes(max_tokens), initialised once with
 * ainfer_moe_workspace_init.
 *
 * ainfer_moe_stack_forward_persistent runs the same L blocks at T <= 4 as one
 * persistent launch (AINFER_ERR_TOKENS above; shapes without a stack
 * geometry, K split of more than 8 waves, return AINFER_ERR_SHAPE).  Its
 * workgroups must all be resident at once: it needs the device to itself
 * (a concurrent kernel turns its waits into bounded time-outs: NaN outputs
 * and AINFER_ERR_SYNC from ainfer_moe_workspace_check).  It is slower than
 * the replayed form on MI355X (c4, T = 1: about 2.6 against 2.0 ms per 60
 * layers); callers that cannot launch from the host per layer are its use.
 * Its workspace holds every layer's intermediates (about 0.5 MB per layer at
 * H4096/E512/k10/I1024, T = 4).  Calls on one workspace must not overlap. */
size_t ainfer_moe_stack_workspace_bytes(const ainfer_moe_shape *shape,
                                        int32_t max_tokens, int32_t n_layers);
size_t ainfer_moe_stack_table_bytes(int32_t n_layers);
/* layers: host array [n_layers] of device weight pointers (validated as in
 * forward); norm_w: host array [n_layers] of device RMSNorm weights ([H]
 * bf16, 16-byte aligned, NULL entries = unit weight), or NULL for all unit.
 * table: device memory of ainfer_moe_stack_table_bytes, 16-byte aligned.
 * Blocks until the table is written (an init-time call). */
int ainfer_moe_stack_prepare(const ainfer_moe_shape *shape,
                             const ainfer_moe_weights *layers,
                             const void *const *norm_w, int32_t n_layers,
                             void *table, size_t table_bytes, void *stream);
int ainfer_moe_stack_forward(const ainfer_moe_shape *shape, const void *table,
                             int32_t n_layers, int32_t norm_mode, float eps,
                             const void *resid_in, void *resid_out, int32_t T,
                             void *workspace, size_t workspace_bytes, void *stream);
int ainfer_moe_stack_forward_persistent(const ainfer_moe_shape *shape, const void *table,
                                        int32_t n_layers, int32_t norm_mode, float eps,
                                        const void *resid_in, void *resid_out, int32_t T,
                                        void *workspace, size_t workspace_bytes,
                                        void *stream);

/* Bytes of the static device scratch behind ainfer_moe_block_forward_noalloc
 * (one copy per GPU the library runs on, held until the process ends). */
#define AINFER_MOE_NOALLOC_SCRATCH_BYTES (16u << 20)

/* ainfer_moe_block_forward without a workspace argument: the workspace is a
 * static device array of AINFER_MOE_NOALLOC_SCRATCH_BYTES per GPU, and the
 * call makes no allocation of any kind (no hipMalloc, no allocating library
 * routine).  It has no counterpart in the reference; it is for callers that
 * cannot allocate: code under HIP graph capture, tight serving loops,
 * harnesses that forbid allocation.  A call whose workspace_bytes(shape, T)
 * exceeds the scratch returns AINFER_ERR_SCRATCH (16 MiB holds, e.g., every
 * decode call up to 16 tokens and H4096/E512/k10/I1024 up to 64 tokens).
 * Every call on one GPU shares that GPU's scratch and starts by zeroing its
 * synchronisation words, so no workspace_init is needed and a wait that ran
 * out in one call (its outputs are NaN) does not affect the next; calls that
 * overlap on one GPU (different streams, or different host threads) race and
 * give wrong results.  Outputs are bit-identical to ainfer_moe_block_forward
 * on the same inputs. */
int ainfer_moe_block_forward_noalloc(const ainfer_moe_shape *shape,
                                     const ainfer_moe_weights *weights,
                                     const void *norm_w, int32_t norm_mode, float eps,
                                     const void *resid_in, void *resid_out, int32_t T,
                                     void *stream);

/* ---- stage-level entries (the pieces forward composes) ----------------- */

/* Router: topk_idx[T][k] int32, topk_w[T][k] fp32 (renormalised, slot 0 =
 * largest logit), shared_gate[T] fp32 (sigmoid, or 1), and optionally
 * logits[T][E] fp32 (NULL to skip).  Workspace as for forward. */
int ainfer_moe_route(const ainfer_moe_shape *shape,
                     const ainfer_moe_weights *weights, const void *x,
                     int32_t T, int32_t *topk_idx, float *topk_w,
                     float *shared_gate, float *logits, void *workspace,
                     size_t workspace_bytes, void *stream);

/* Dispatch (T <= AINFER_MOE_CHUNK_TOKENS): counts[E], offsets[E+1] (exclusive scan of counts),
 * perm[T*k] (position p holds t*k + j, expert-contiguous, token ascending
 * within an expert) and inv_perm[T*k] (inverse of perm).  Each row of
 * topk_idx must hold k distinct expert ids in [0, E), as ainfer_moe_route
 * writes them; the contents are not checked (other values are undefined
 * behaviour, including out-of-bounds device accesses). */
int ainfer_moe_dispatch(const ainfer_moe_shape *shape,
                        const int32_t *topk_idx, int32_t T, int32_t *counts,
                        int32_t *offsets, int32_t *perm, int32_t *inv_perm,
                        void *workspace, size_t workspace_bytes, void *stream);

/* Expert stage alone (W4A16, T <= AINFER_MOE_CHUNK_TOKENS), for routing the
 * caller computed (ainfer_moe_route or its own; topk_idx as for
 * ainfer_moe_dispatch: k distinct ids in [0, E) per row, not checked): o[T*k + T][H] bf16, 16-byte
 * aligned; row t*k + j is expert topk_idx[t][j] applied to token t (gate/up,
 * SiLU-mul, down), row T*k + t the shared expert on token t (unused without
 * one).  The kernels and arithmetic of ainfer_moe_forward's expert stage at
 * the same T (for T <= 2 forward fuses the stages and splits K differently;
 * there the rows agree within the layer tolerance).  No reference counterpart
 * (the reference is dense); the per-expert MLP is decode_l0.cpp:663-674's. */
int ainfer_moe_experts(const ainfer_moe_shape *shape,
                       const ainfer_moe_weights *weights, const void *x,
                       const int32_t *topk_idx, int32_t T, void *o,
                       void *workspace, size_t workspace_bytes, void *stream);

/* Combine: y[t] = bf16(sum_j topk_w[t][j] * o[t*k + j] + shared_gate[t] *
 * o[T*k + t] (+ resid[t])), fp32 fma in slot order, as ainfer_moe_forward;
 * o as ainfer_moe_experts writes it, resid NULL or [T][H] bf16 (the residual
 * add of ResAddF, kernels.cpp:646-652).  16-byte aligned rows. */
int ainfer_moe_combine(const ainfer_moe_shape *shape, const void *o,
                       const float *topk_w, const float *shared_gate,
                       const void *resid, void *y, int32_t T, void *stream);

/* RMSNorm over rows: y[T][H] bf16 = x * 1/sqrt(mean(x^2) + eps) * w
 * (norm_mode PLAIN) or * (1 + w) (ONE_PLUS); w bf16 [H] or NULL (unit).
 * Sum of squares in fp64, as RMSNormW (kernels.cpp:73-116). */
int ainfer_moe_rmsnorm(const void *x, const void *w, int32_t norm_mode,
                       float eps, void *y, int32_t T, int32_t H, void *stream);

/* ---- .binfer containers ---------------------------------------------------
 * The reference's v1 container (docs/binfer_spec.md): header, section table,
 * identity / architecture / tokenizer / policy sections, tensor directory,
 * scale pool, 64-byte aligned payloads, trailing SHA-256.  An MoE layer l is
 * the tensors model.layers.<l>.mlp.{gate.weight [E][H] bf16, gate.bias [E]
 * fp32 (optional), shared_expert_gate.weight [1][H] bf16 (optional),
 * experts.{gate,up}_proj.weight [E][I][H] and experts.down_proj.weight
 * [E][H][I] (INT4, layout_id AINFER_BINFER_LAYOUT_EXPERTS),
 * shared_expert.{gate,up,down}_proj.weight (INT4, row-major)} and
 * model.layers.<l>.post_attention_layernorm.weight [H] bf16 (optional); the
 * architecture section (JSON) holds hidden, n_experts, top_k, inter,
 * shared_inter, layers, scale_fp16 and rms_eps.  ainfer_amd/binfer.py writes
 * such files.
 * Additions in fields v1 reserves: layout_id AINFER_BINFER_LAYOUT_EXPERTS (in
 * the experimental range, which v1 reference loaders reject) = E stacked
 * row-major [rows][K] matrices, the weight layout of this ABI; byte 180 of a
 * directory entry = scale dtype of an INT4 tensor (0 bf16, the v1 default;
 * 1 fp16). */
#define AINFER_BINFER_LAYOUT_EXPERTS 32
typedef struct ainfer_binfer ainfer_binfer;
/* Open and validate the whole file before anything is allocated: magic,
 * version, flags, section CRCs, directory size and CRC, unique names, no
 * visual tensors, known dtypes and layout ids, quantization sizes, bounds,
 * overlaps, payload CRCs and the trailing SHA-256 (the reference loader's
 * rules, docs/binfer_spec.md:112-116, tools/binfer.py:383-499).  On failure
 * returns AINFER_ERR_FORMAT (or AINFER_ERR_IO) and writes the first failure,
 * with the tensor name and expected/actual values, into err. */
int ainfer_binfer_open(const char *path, ainfer_binfer **file, char *err, size_t err_len);
void ainfer_binfer_close(ainfer_binfer *file);
/* Text of the last load failure on the file. */
const char *ainfer_binfer_error(const ainfer_binfer *file);
/* The MoE shape, layer count and RMSNorm eps of the architecture section. */
int ainfer_binfer_moe_info(const ainfer_binfer *file, ainfer_moe_shape *shape,
                           int32_t *n_layers, float *eps);
/* Device bytes one layer's tensors take in an arena (each 256-byte aligned). */
size_t ainfer_binfer_moe_layer_bytes(const ainfer_binfer *file, int32_t layer);
/* Check layer `layer`'s tensors against the MoE shape (names, dtypes,
 * layouts, shapes, scale dtype), copy them into the caller's device arena
 * (256-byte aligned, ainfer_binfer_moe_layer_bytes) and fill the weight pointers
 * (and *norm_w, NULL when the file has no norm weight).  Blocks until the
 * copies are done (an init-time call). */
int ainfer_binfer_load_moe_layer(const ainfer_binfer *file, int32_t layer, void *arena,
                                 size_t arena_bytes, ainfer_moe_weights *weights,
                                 const void **norm_w, void *stream);

/* ---- W4A8: the reference's production GEMV numerics ---------------------
 * Activations quantised per group of 128 to int8, INT4 weights, int32 group
 * dots, fp32 rescale in group order.  These two entries are the operator
 * surface of the reference's decode GEMV stage; the MoE layer entries above
 * keep bf16 activations (W4A16). */
enum { AINFER_ACT_F32 = 0, AINFER_ACT_BF16 = 1 };

/* Per-group int8 quantisation of x[T][K] (fp32 or bf16, K % 128 == 0):
 * sq[t][g] = max|x| / 127 over the group (1 when that is 0) and
 * q[t][k] = (int)(x/sq + 0.5) for x/sq >= 0, (int)(x/sq - 0.5) otherwise,
 * clamped to [-127, 127] (round half away from zero).  NaN inputs give
 * unspecified codes.  x 8-byte aligned, q 2-byte aligned.
 * Replaces ScalesMax + Quantize, tools/cmdlist/kernels.cpp:551-579
 * (launched per vector by decode_l0.cpp:505-515). */
int ainfer_moe_act_quant_i8(const void *x, int32_t x_dtype, int32_t T, int32_t K,
                            int8_t *q, float *sq, void *stream);

/* INT4 x int8 GEMV: y[t][m] (fp32) = sum over g = 0..K/128-1, in order, of
 * float(gs) * s[m][g] * sq[t][g], gs = sum_j w[m][128g+j] * q[t][128g+j]
 * exact in int32; products and sums rounded to fp32 one at a time (no fused
 * multiply-add), so y is bit-identical to that formula.  packed [M][K/2]
 * (low nibble = even k), scales [M][K/128] (AINFER_SCALE_BF16 as the
 * reference, or FP16), q [T][K], sq [T][K/128].  packed, q 16-byte aligned.
 * Replaces Int4Gemv(float* Y, const u8* P, const u16* S, const i8* XQ,
 * const float* SQ, int K), tools/cmdlist/kernels.cpp:148-201, bound by
 * decode_l0.cpp:494-504 (one launch per token there; T tokens here). */
int ainfer_moe_int4_gemv_i8(const uint8_t *packed, const void *scales,
                            int32_t scale_dtype, const int8_t *q, const float *sq,
                            int32_t M, int32_t K, int32_t T, float *y, void *stream);

/* Test hook: the number of polls a bounded device-side wait of the decode
 * path makes before it gives up (default 2^20, about 10 ms).  0 makes every
 * such wait give up at once, so tests can drive the timeout path while every
 * kernel still exits normally.  Process-wide; no reference counterpart. */
int ainfer_moe_debug_spin_limit(int32_t polls);

/* Strict mode (process-wide, off by default; no reference counterpart): when
 * on, ainfer_moe_forward, _block_forward, _block_forward_noalloc,
 * _stack_forward and _stack_forward_persistent wait for the stream after
 * enqueueing their work and return AINFER_ERR_SYNC when a bounded device-side
 * wait of the call (or of an earlier call on the same workspace, whose error
 * word is sticky until ainfer_moe_workspace_init) ran out, instead of
 * AINFER_OK with NaN rows.  For validation runs and callers that read the
 * result at once anyway; it costs a host round trip per call.  Under HIP
 * graph capture the check is skipped (nothing can be waited for there). */
int ainfer_moe_set_strict(int32_t on);

/* ---- synthetic data (counter-based, bit-identical to the CPU oracle) --- */
enum {
  AINFER_FILL_BYTES = 0,      /* uniform random bytes (packed int4 weights)  */
  AINFER_FILL_BF16_NORMAL = 1,/* bf16 of std * n,  n ~ standardised sum of
                                 8 uniform bytes (Irwin-Hall approximation of
                                 N(0,1))                                     */
  AINFER_FILL_FP16_ABSNORMAL = 2, /* fp16 of |std * n|                       */
  AINFER_FILL_BF16_ABSNORMAL = 3  /* bf16 of |std * n|                       */
};
/* Fill n elements (bytes for FILL_BYTES, 2-byte values otherwise) of out.
 * Element i is a function of (seed, i) only. */
int ainfer_moe_fill(int32_t kind, uint64_t seed, float std_, size_t n,
                    void *out, void *stream);

/* ---- per-stage timing (the AINFER_PROFILE instrumentation of
 * tools/decode/decode_l0.cpp:705,714-725,870-884, with device events) -----
 * While enabled, forward/block_forward record a HIP event on the caller's
 * stream before and after every kernel.  For T <= 16 stage 2 is the routing
 * kernel (logits, top-k, weights, dispatch) and stages 1 and 3 read 0; at
 * T = 1 stage 5 is the down + combine kernel (stage 4 the gate/up kernel) and
 * at T = 2 the fused expert kernel (gate/up, down and combine), with stage 6
 * (and at T = 2 stage 4) reading 0.  ainfer_moe_profile_read()
 * waits for them and returns, per stage, the mean device time in
 * microseconds over the calls since enable, and the call count.  Stages:
 * 0 rmsnorm, 1 router, 2 top-k (+ dispatch when T <= 64), 3 dispatch,
 * 4 gate/up, 5 down, 6 combine. */
#define AINFER_MOE_N_STAGES 7
int ainfer_moe_profile_enable(int32_t enable);
int ainfer_moe_profile_read(float *stage_us, int32_t n_stages, int32_t *n_calls);
/* Mean duration of the decode gate/up kernel itself over the calls since
 * enable (T <= 16 paths with a gate/up launch of its own): while profiling,
 * that launch goes through hipExtLaunchKernel with start/stop events stamped
 * by the dispatch, so the figure carries no event-packet overhead and is
 * what a kernel trace reports.  No counterpart in the reference: a
 * measurement aid for roofline figures. */
int ainfer_moe_profile_kernel(float *gate_up_us, int32_t *n_launches);

/* The MFMA ceiling of a main loop: every wave of one block per CU
 * (waves_per_simd in 1..4 per SIMD) issues iters x 16 independent
 * v_mfma_f32_16x16x32_bf16 with valu_per_mfma (0..4) independent fp32 FMAs
 * after each; *tflops receives the bf16 MFMA rate of the second of two
 * launches on `stream` (host-synchronous).  No counterpart in the reference:
 * a measurement aid for the prefill GEMM's roofline. */
int ainfer_moe_mfma_probe(int32_t valu_per_mfma, int32_t waves_per_simd, int32_t iters,
                          void *stream, float *tflops);

/* The sustainable HBM read rate: iters launches of a read-only kernel that
 * walks `bytes` of `buf` (16-byte aligned, a multiple of 16; fill it with
 * random bytes, not a uniform value) with `unroll`
 * (1, 2, 4, 8 or 16) independent 16-byte loads in flight per lane, on
 * blocks_per_cu x CUs blocks of 256 threads; *gbs receives bytes x iters over
 * the elapsed time on `stream` (host-synchronous).  The buffer is a probe
 * buffer: its first 16 bytes receive a lane's fold in the (2^-128 per lane)
 * case that the fold is all ones.  No counterpart in the
 * reference's operator surface: the read roof its own tuning measured before
 * any kernel (tasks.md:240-250), for decode's "fraction of measured". */
int ainfer_moe_read_probe(const void *buf, uint64_t bytes, int32_t unroll, int32_t blocks_per_cu,
                          int32_t iters, void *stream, float *gbs);

#ifdef __cplusplus
}
#endif
#endif /* AINFER_MOE_H */
