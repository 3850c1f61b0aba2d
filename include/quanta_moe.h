/*
 * quanta_moe.h -- C ABI of the MI355X (gfx950) quantized sparse-MoE block.
 *
 * The reference (pmrjge/quanta) has no native boundary: its block is the Python function
 * qwen35_moe (src/quanta/qwen35/moe.py:154-202) over MLX primitives (mx.gather_qmm,
 * mx.argpartition, mx.argsort, mx.softmax, mx.dequantize). Each entry point below replaces
 * one of those steps; the citation names the reference line it stands in for. The Python
 * mirror of the reference surface (quanta_amd.moe.qwen35_moe / Qwen35MoEModule) binds these
 * symbols with ctypes.
 *
 * Conventions (all entry points):
 *  - Every pointer is a DEVICE pointer owned by the caller; the library never allocates.
 *    Scratch memory comes from the caller through `ws` (size from qmoe_forward_workspace).
 *  - `stream` is a hipStream_t (NULL = the default stream). Calls enqueue work and return
 *    without synchronising the host.
 *  - Return value: QMOE_OK (0), QMOE_EINVAL (-1, bad argument, nothing enqueued) or
 *    QMOE_EHIP (-2, HIP launch error). qmoe_last_error() holds a thread-local message.
 *  - bf16 tensors are passed as uint16_t bit patterns, packed int4 codes as uint32 words.
 *  - Calls on different streams are independent; calls sharing workspace must be ordered by
 *    the caller. Library state: the thread-local error string, and for qmoe_forward one
 *    auxiliary stream per device (default priority, created with its events on first use)
 *    that runs independent parts of the block concurrently, forked from and joined back into
 *    `stream` with events; a mutex serialises the enqueue of concurrent calls.
 */
#ifndef QUANTA_MOE_H_
#define QUANTA_MOE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QMOE_ABI_VERSION 10

#define QMOE_OK 0
#define QMOE_EINVAL (-1)
#define QMOE_EHIP (-2)

/* scoring functions (cfg.scoring_func, src/quanta/qwen35/config.py:129) */
#define QMOE_SCORE_SOFTMAX 0
#define QMOE_SCORE_SIGMOID 1
#define QMOE_SCORE_SQRTSOFTPLUS 2   /* DeepSeek-V4: sqrt(softplus(logit)), src/quanta/dsv4/moe.py:37-57 */

/* renormalisation of the k routing weights, w /= sum(w) + 1e-20 (the config's norm_topk):
 *  NONE    never
 *  ALWAYS  whenever set, k = 1 included (qwen35_route, src/quanta/qwen35/moe.py:53-54; DeepSeek-V4
 *          renormalises its non-softmax scores unconditionally, src/quanta/dsv4/moe.py:54-55)
 *  MULTI   only when k > 1 (the sigmoid + correction-bias MoEGate routers,
 *          src/quanta/modeling/moe.py:41-42, src/quanta/glm/moe.py:53-54,
 *          src/quanta/minimax/moe.py:54-55: a single expert keeps its score) */
#define QMOE_NORM_NONE 0
#define QMOE_NORM_ALWAYS 1
#define QMOE_NORM_MULTI 2

/* expert weight formats, both in this library's MFMA-tiled layout (see qmoe_tile_*) */
#define QMOE_FMT_INT4_G64 0
#define QMOE_FMT_BF16 1
#define QMOE_FMT_INT6_G64 2 /* affine int6 codes, bf16 scale/bias per 64 (MiniMax M3 experts,
                               src/quanta/minimax/model_m3.py:414-450); the large regime needs
                               row exponents, as int4 */
#define QMOE_FMT_INT3_G64 3 /* affine int3 codes, bf16 scale/bias per 64 (Kimi's int3 gate/up
                               stacks, src/quanta/modeling/quantized.py:1-84); the large regime
                               needs row exponents, as int4 */
#define QMOE_FMT_INT8_G64 4 /* affine int8 codes, bf16 scale/bias per 64: the shared expert as the
                               bake stores it (src/quanta/qwen35/bake.py:147-151); shared expert
                               only (qmoe_config_t.shared_format) and qmoe_grouped_qmm's small
                               regime */

/* router weight storage */
#define QMOE_ROUTER_BF16_TILED 0 /* bf16 [router_rows, H] tiled; row E = shared-expert gate */
#define QMOE_ROUTER_F32 1        /* fp32 row-major [E, H]; shared gate fp32 [H] separately */

/* grouped-qmm regimes */
#define QMOE_REGIME_AUTO 0
#define QMOE_REGIME_SMALL 1 /* 16-token m-tiles, weights streamed to registers (decode) */
#define QMOE_REGIME_LARGE 2 /* prefill: experts of > 16 rows on 128-row LDS-staged fp16 tiles
                               (128x512 for int4 weights in 512-row blocks, else 128x256),
                               the others on 16-token m-tiles */

/* gated activation of the SwiGLU epilogue, h = act(gate, up) on the bf16 gate/up values in fp32:
 *  SILU        silu(g) * u                                (src/quanta/qwen35/moe.py:59-63)
 *  SILU_CLAMP  silu(min(g, L)) * clip(u, -L, L)           (src/quanta/dsv4/moe.py:74-77, L = swiglu_limit)
 *  SWIGLU_OAI  (clip(u, -L, L) + 1) * g' * sigmoid(alpha * g'), g' = min(g, L)
 *                                                         (src/quanta/minimax/model_m3.py:112-128,
 *                                                          alpha 1.702, L 7.0) */
#define QMOE_ACT_SILU 0
#define QMOE_ACT_SILU_CLAMP 1
#define QMOE_ACT_SWIGLU_OAI 2

/* grouped-qmm epilogues */
#define QMOE_EPI_SWIGLU 0 /* out[:, j] = bf16(silu(bf16(gate_j)) * bf16(up_j)), rows = [gate; up] */
#define QMOE_EPI_BF16 1
#define QMOE_EPI_F32 2

/* Block configuration. Mirrors Qwen35Config's MoE fields (src/quanta/qwen35/config.py:125-130)
 * plus the DeepSeek/GLM router fields (n_group, topk_group, routed_scaling_factor,
 * src/quanta/glm/config.py:65,69). */
typedef struct {
  int32_t hidden;        /* H, multiple of 256 */
  int32_t n_experts;     /* E <= 1024 */
  int32_t top_k;         /* k (num_experts_per_tok or topk_override), 1 <= k <= min(E, 64) */
  int32_t inter;         /* I, multiple of 128 */
  int32_t shared_inter;  /* Is, 0 = no shared expert, else multiple of 128 */
  int32_t scoring;       /* QMOE_SCORE_* */
  int32_t norm_topk;     /* QMOE_NORM_*: renormalise the k weights, w /= sum(w) + 1e-20 */
  int32_t n_group;       /* expert groups (1 = plain top-k) */
  int32_t topk_group;    /* groups kept when n_group > 1 */
  float routed_scale;    /* routed_scaling_factor applied after renormalisation */
  int32_t expert_format; /* QMOE_FMT_* */
  int32_t router_format; /* QMOE_ROUTER_* */
  int32_t router_rows;   /* rows of the tiled bf16 router (>= E + shared_gated, % 256 == 0) */
  int32_t shared_gated;  /* 1: shared output scaled by sigmoid(x . shared_expert_gate) */
  int32_t regime;        /* QMOE_REGIME_* for the routed experts (AUTO: small for N <= 256) */
  int32_t act;           /* QMOE_ACT_* of the routed and shared experts' SwiGLU */
  float act_alpha;       /* SWIGLU_OAI's alpha */
  float act_limit;       /* SILU_CLAMP / SWIGLU_OAI's clamp L (> 0; +inf = none) */
  int32_t down_format;   /* QMOE_FMT_* of the routed down projection (gate_up: expert_format);
                            both quantized or both bf16 (Kimi: gate/up int3, down int4,
                            src/quanta/modeling/quantized.py:4-7) */
  int32_t awq;           /* 1: the quantized experts carry activation-aware scales (weights'
                            awq_gu / awq_dn, DeepSeek-V4, src/quanta/dsv4/moe.py:112-137): the
                            activation is divided by the expert's per-input-channel scale before
                            each projection; the large regime needs inter % 256 == 0 (else
                            the small regime runs every batch size) */
  int32_t mixed;         /* 1: routed experts of mixed widths per (expert, projection), passed to
                            qmoe_forward_mixed; both regimes (above 256 tokens every stack needs
                            qmoe_stack_t.row_exp). The weights' gu/dn fields are then unused and
                            expert_format / down_format are placeholders (any pair the config
                            check accepts, bf16 included): the stacks' formats pick every
                            kernel */
  int32_t shared_format; /* QMOE_FMT_BF16 or QMOE_FMT_INT8_G64: the shared expert's weights.
                            int8 weights are dequantized in registers to bf16(s*q + b), the bf16
                            weights the reference's loader makes of them
                            (src/quanta/qwen35/artifact.py:105-115), so both formats give the same
                            outputs; int8 reads half the bytes. Above 256 tokens the block first
                            expands them into its workspace. */
} qmoe_config_t;

/* Prepared (resident) weights of one block; every array is device memory. */
typedef struct {
  const void* router_w;           /* see router_format */
  const float* router_bias;       /* [E] e_score_correction_bias (selection only) or NULL */
  const float* shared_gate_w;     /* [H] fp32, only with QMOE_ROUTER_F32 */
  const uint32_t* gu_codes;       /* routed gate|up [E, 2I, H]: tiled int3/int4/int6 codes
                                     (qmoe_tile_int3/int4/int6) or tiled bf16 */
  const uint16_t* gu_sb;          /* tiled scale/bias (quantized formats only) */
  const uint32_t* dn_codes;       /* routed down [E, H, I] */
  const uint16_t* dn_sb;
  const uint16_t* sh_gu;          /* shared gate|up [2*Is, H]: tiled bf16, or tiled int8 codes
                                     (qmoe_tile_int8) with shared_format QMOE_FMT_INT8_G64 */
  const uint16_t* sh_dn;          /* shared down [H, Is], as sh_gu */
  const uint16_t* sh_gu_sb;       /* int8 shared expert: tiled scale/bias of sh_gu, else unused */
  const uint16_t* sh_dn_sb;       /* int8 shared expert: tiled scale/bias of sh_dn, else unused */
  const uint16_t* awq_gu;         /* config awq: bf16 [E, 2, H] input-channel scales of the gate
                                     (row 0) and up (row 1) projections, else NULL */
  const uint16_t* awq_dn;         /* config awq: bf16 [E, I] scales of the down projection */
  const int8_t* gu_rexp;          /* int3/int4/int6 gate|up: per weight row [E, 2I] power-of-two
                                     exponent (qmoe_row_exponents) for the prefill kernels' fp16
                                     dequant; required when a call reaches the large regime
                                     (N > 256), may be NULL for decode-only use */
  const int8_t* dn_rexp;          /* int3/int4/int6 down: per weight row [E, H], as gu_rexp */
} qmoe_weights_t;

int qmoe_abi_version(void);
const char* qmoe_last_error(void);

/* Whole block: y[N,H] = bf16(sum_s w[t,s] * expert_{idx[t,s]}(x[t]) + shared(x[t])).
 * Replaces qwen35_moe (src/quanta/qwen35/moe.py:154-202) for one token chunk: router
 * (:178), packed routed SwiGLU via two gather_qmm (:85-124, :189), fp32 combine (:191),
 * gated shared expert (:145-151, :201) and the bf16 cast (:202). N <= 65535. */
size_t qmoe_forward_workspace(const qmoe_config_t* cfg, int64_t N);
int qmoe_forward(const qmoe_config_t* cfg, const qmoe_weights_t* w, const uint16_t* x, int64_t N,
                 uint16_t* y, void* ws, size_t ws_bytes, void* stream);

/* qmoe_forward without allocation, for callers that cannot allocate: code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc. No counterpart in the reference
 * (MLX allocates inside its lazy graph). The workspace is a fixed device array inside the library,
 * QMOE_NOALLOC_SCRATCH_BYTES (64 MiB) on each GPU the library runs on, held until the process
 * ends; calls whose qmoe_forward_workspace exceeds it are refused (QMOE_EINVAL). Every launch
 * goes on `stream` (no auxiliary stream or events are created). The call allocates nothing: no
 * hipMalloc/hipFree, no allocating library routine. Calls that overlap on one GPU race on the
 * shared scratch: order them on one stream. Same outputs as qmoe_forward, bit for bit. */
#define QMOE_NOALLOC_SCRATCH_BYTES (64u << 20)
int qmoe_forward_noalloc(const qmoe_config_t* cfg, const qmoe_weights_t* w, const uint16_t* x,
                         int64_t N, uint16_t* y, void* stream);

/* Decode dataflow launch (tuning and diagnostics; no counterpart in the reference, whose MLX
 * graph schedules its primitives itself). Decode batches routed slot-major, with int4 experts, a
 * bf16 router and a shared expert, can run everything after the router launch (top-k, routed
 * gate_up and down, shared down, combine) as one launch whose units wait on each other through
 * counters in the workspace; the outputs equal the multi-launch path's bit for bit.
 * Mode 1 (the default) takes it for one- and two-token calls, where it is the faster path;
 * qmoe_set_decode_flow(0) makes later calls launch the stages one by one, (2) takes the single
 * launch for every batch it covers (up to the slot-major sizes; for tests and measurements). It
 * returns the previous mode (process-wide, not thread-safe against calls in flight).
 * qmoe_flow_timeouts() returns how many in-kernel waits (this launch's and the routing tail's,
 * below) have run out of their bound on the current device since the library loaded (0 in a
 * healthy run; synchronous). */
int qmoe_set_decode_flow(int mode);
uint32_t qmoe_flow_timeouts(void);

/* Routing tail (tuning; no counterpart in the reference, whose MLX graph schedules its
 * primitives itself). Decode batches of up to 64 tokens sorted by expert, with a bf16 router and
 * a shared expert in the router launch, rank their tokens in that launch's last router
 * workgroups and sort the slots in the last of them, instead of the top-k and permute launches;
 * the outputs are the same bit for bit. On (1) by default; qmoe_set_route_tail(0) makes later
 * calls use the separate launches. Returns the previous setting (process-wide; other values
 * change nothing). */
int qmoe_set_route_tail(int on);

/* Routed experts whose widths vary per (expert, projection) (Kimi's QuantizedSparseMoE,
 * src/quanta/modeling/quantized.py:40-84: one packed stack per projection and width, each expert
 * carrying per projection its width and its slot in that width's stack). Each stack is tiled as
 * the uniform stacks (qmoe_tile_int3/int4/int6; gate and up [E_w, I, H], down [E_w, H, I]) and
 * names, per expert, the slot it holds in the stack or -1. Every expert must be in exactly one
 * stack per projection (the library cannot check the device maps). The gate and up projections
 * are separate stacks, as in the reference. */
#define QMOE_PROJ_GATE 0
#define QMOE_PROJ_UP 1
#define QMOE_PROJ_DOWN 2
#define QMOE_PROJ_GATE_UP 3   /* gate and up fused per width ([E_w, 2I, H], gate rows first), when
                                 every expert's gate and up share width and slot; then no GATE or
                                 UP stacks */
#define QMOE_MAX_STACKS 12
typedef struct {
  int32_t proj;                /* QMOE_PROJ_* */
  int32_t format;              /* QMOE_FMT_INT3_G64 / INT4_G64 / INT6_G64 */
  const uint32_t* codes;       /* tiled codes */
  const uint16_t* sb;          /* tiled scale/bias */
  const int32_t* expert_slot;  /* [E] device: the expert's slot in this stack, or -1 */
  const int8_t* row_exp;       /* [E_w][rows] device (qmoe_row_exponents of the stack): needed
                                  in the large regime (N > 256), else may be NULL */
} qmoe_stack_t;
typedef struct {
  int32_t n_stacks;            /* 2 .. QMOE_MAX_STACKS, every projection at least once */
  qmoe_stack_t stacks[QMOE_MAX_STACKS];
} qmoe_mixed_t;

/* qmoe_forward with the routed experts of mixed widths (cfg->mixed = 1); workspace as
 * qmoe_forward_workspace. Replaces QuantizedSparseMoE.__call__ (src/quanta/modeling/
 * quantized.py:68-84): gate and up by width (fused per width with the SwiGLU epilogue when a
 * QMOE_PROJ_GATE_UP stack holds them, else into one [N*k, 2I] buffer and h = bf16(silu(g) * u)),
 * then down by width. */
int qmoe_forward_mixed(const qmoe_config_t* cfg, const qmoe_weights_t* w, const qmoe_mixed_t* mixed,
                       const uint16_t* x, int64_t N, uint16_t* y, void* ws, size_t ws_bytes,
                       void* stream);

/* The block with the decoder layer's steps either side of it, as the layer calls it:
 *   y = bf16(x + bf16(block(rmsnorm(x))))
 * Replaces post_attention_layernorm -> mlp -> residual add, x = x + mlp(
 * post_attention_layernorm(x)) (src/quanta/qwen35/model.py:104-105; the batched decode step
 * src/quanta/qwen35/batched_runtime.py:304-306). rmsnorm(x) = bf16(norm_w * (x * rsqrt(mean(x^2)
 * + eps))) in fp32, norm_w [H] bf16 being nn.RMSNorm's resident weight (source weight + 1,
 * src/quanta/qwen35/runtime.py:57-63). The normalised rows live in the workspace; the residual
 * add is fused into the block's final combine; y may alias x. */
size_t qmoe_forward_residual_workspace(const qmoe_config_t* cfg, int64_t N);
int qmoe_forward_residual(const qmoe_config_t* cfg, const qmoe_weights_t* w, const uint16_t* x,
                          const uint16_t* norm_w, float eps, int64_t N, uint16_t* y, void* ws,
                          size_t ws_bytes, void* stream);

/* ---- the block at the reference's own dtypes and group sizes ----
 * qmoe_forward requires bf16 activations, bf16 scale/bias, group 64/128 and dimensions that are
 * multiples of 128. The reference's block takes any float dtype the caller baked: its
 * packed-expert parity gate (parity/qwen35_forward_test.py:213-271) runs float32 activations
 * with float32 scale/bias, int4 group 32, hidden 32 and moe_intermediate 64, and its
 * sparse-vs-dense gate (parity/qwen35_forward_test.py:192-209) float32 dense stacks at
 * moe_intermediate 16. qmoe_forward_general runs those, following the reference's dtype flow
 * (src/quanta/qwen35/moe.py:36-56, 66-124, 145-151, 154-202):
 *   logits = f32(x) @ f32(gate)^T (+ column E = the shared gate logit); top-k as qmoe_router_topk
 *   routed experts in dtype T: a dense stack's dtype (x cast to it), or for packed codes the
 *     promotion of x's and the scales' dtypes (f32 if either is); gate_up, SwiGLU, down each
 *     rounded to T; codes any width 2..6 or 8, LSB-first bitstream rows, groups 32/64/128
 *   routed = sum_s f32(d) * w;  shared = f32(down(glu(xs Wg^T, xs Wu^T))) * sigmoid(f32(x) .
 *     f32(shared_expert_gate)), xs = x cast to the shared weights' dtype
 *   y = cast to x's dtype (routed + shared)
 * Every product accumulates in fp32 with one wavefront per output value; a matvec kernel for
 * small and odd shapes, not the production path. dense_all = 1 is the run-every-expert form
 * (qwen35_moe(sparse=False), src/quanta/qwen35/moe.py:127-142; dense stacks only). */
#define QMOE_DT_BF16 0
#define QMOE_DT_F32 1

typedef struct {
  int32_t hidden, n_experts, top_k, inter, shared_inter;  /* shared_inter 0: no shared expert */
  int32_t scoring, norm_topk, n_group, topk_group;        /* as qmoe_config_t */
  float routed_scale;
  int32_t act;                /* QMOE_ACT_* with act_alpha, act_limit as in qmoe_config_t */
  float act_alpha, act_limit;
  int32_t x_dtype;            /* QMOE_DT_* of x and y */
  int32_t gate_dtype;         /* router weight [E, H] */
  int32_t experts_packed;     /* 1: affine codes + scale/bias; 0: dense stacks */
  int32_t expert_dtype;       /* dense stacks' dtype, or the packed scale/bias dtype */
  int32_t bits, group_size;   /* packed codes: 2..6 or 8 bits, groups of 32, 64 or 128 */
  int32_t shared_dtype;       /* shared gate/up/down weights */
  int32_t shared_gated;       /* 1: sh_expert_gate [1, H] scales the shared expert */
  int32_t shared_gate_dtype;
  int32_t dense_all;          /* 1: run every expert (sparse=False) */
} qmoe_general_config_t;

typedef struct {
  const void* gate;           /* [E, H] */
  const float* router_bias;   /* [E] correction bias for selection, or NULL */
  const void* gu;             /* packed [E, 2I, H*bits/32] uint32, or dense [E, 2I, H] */
  const void* gu_scale;       /* [E, 2I, H/gs] (packed only) */
  const void* gu_bias;
  const void* dn;             /* packed [E, H, I*bits/32], or dense [E, H, I] */
  const void* dn_scale;       /* [E, H, I/gs] */
  const void* dn_bias;
  const void* sh_gate;        /* [Is, H] */
  const void* sh_up;          /* [Is, H] */
  const void* sh_down;        /* [H, Is] */
  const void* sh_expert_gate; /* [1, H] */
} qmoe_general_weights_t;

size_t qmoe_forward_general_workspace(const qmoe_general_config_t* cfg, int64_t N);
int qmoe_forward_general(const qmoe_general_config_t* cfg, const qmoe_general_weights_t* w,
                         const void* x, int64_t N, void* y, void* ws, size_t ws_bytes,
                         void* stream);

/* RMSNorm rows alone (the same arithmetic as qmoe_forward_residual's norm):
 * out[t] = bf16(w * (x[t] * rsqrt(mean(x[t]^2) + eps))), fp32 math, H % 8 == 0. Replaces
 * nn.RMSNorm / mx.fast.rms_norm as the reference restates it (src/quanta/qwen35/
 * attention.py:113-117; src/quanta/qwen35/mtp.py:40-42). */
int qmoe_rmsnorm(const uint16_t* x, const uint16_t* w, int64_t N, int H, float eps, uint16_t* out,
                 void* stream);

/* Top-k selection from router logits [N, ld_logits] (fp32): softmax or sigmoid scores,
 * optional correction bias [E] for selection, group-limited selection when n_group > 1,
 * renormalisation (norm_topk: QMOE_NORM_*, +1e-20) and routed_scale. Outputs idx[N,k] (int32, canonical order:
 * choice value descending, id ascending) and w[N,k] (fp32). With has_shared_gate, column E
 * holds the shared-gate logit and shared_gate_out[N] = sigmoid(logit).
 * Replaces qwen35_route (src/quanta/qwen35/moe.py:36-56) and MoEGate.__call__
 * (src/quanta/modeling/moe.py:33-44; src/quanta/glm/moe.py:44-55). */
int qmoe_router_topk(const float* logits, int64_t ld_logits, const float* bias, int64_t N, int E,
                     int k, int scoring, int n_group, int topk_group, int norm_topk,
                     float routed_scale, int has_shared_gate, int32_t* idx, float* w,
                     float* shared_gate_out, void* stream);

/* The router in one call, from the gate weight as the artifact stores it: wr [E, H] row-major,
 * bf16 (wr_is_f32 = 0, the bake's dtype, src/quanta/qwen35/bake.py:147-148) or fp32
 * (wr_is_f32 = 1). logits = x . wr^T in fp32 (bf16 x bf16 products are exact in fp32), then the
 * top-k of qmoe_router_topk: idx[N,k] int32 in canonical order, w[N,k] fp32. shared_gate
 * (nullable; [H], wr's dtype) adds the shared-expert gate: shared_gate_out[N] =
 * sigmoid(x . shared_gate). The logits live in `ws` (qmoe_router_workspace bytes). x, wr and
 * shared_gate 16-byte aligned, H % 8 == 0, N <= 262140 per call.
 * Replaces qwen35_route(xf, gate_w, cfg) (src/quanta/qwen35/moe.py:36-56) and MoEGate.__call__
 * (src/quanta/modeling/moe.py:33-44) taking the raw gate, with no tiling step. */
size_t qmoe_router_workspace(int64_t N, int E);
int qmoe_router(const uint16_t* x, const void* wr, int wr_is_f32, const void* shared_gate,
                const float* bias, int64_t N, int H, int E, int k, int scoring, int n_group,
                int topk_group, int norm_topk, float routed_scale, int32_t* idx, float* w,
                float* shared_gate_out, void* ws, size_t ws_bytes, void* stream);

/* Router logits for an fp32 router weight [E,H] (row-major): logits[t, e] = x[t] . wr[e] in
 * fp32; column E = x[t] . shared_gate when shared_gate != NULL. Replaces the fp32 matmul
 * xf.astype(f32) @ gate_w.astype(f32).T (src/quanta/qwen35/moe.py:47). bf16 routers go through
 * qmoe_grouped_qmm with QMOE_EPI_F32 (products of bf16 are exact in fp32). */
int qmoe_router_logits_f32(const uint16_t* x, const float* wr, const float* shared_gate,
                           int64_t N, int H, int E, float* logits, int64_t ld_logits,
                           void* stream);

/* Stable permute of the N*k (token, slot) pairs by expert id. Outputs counts[E],
 * offsets[E+1], tile_off[E+1] (prefix of ceil(count/m_tile)), sorted_slot[N*k]
 * (sorted position -> slot t*k+s) and inv[N*k] (slot -> sorted position, -1 for ids outside
 * [0,E)). Requires distinct experts within each token (true of any top-k router).
 * Optional tile_map (int32 x4 per m-tile, max_tiles >= ceil(N*k/m_tile) + min(E, N*k)) receives
 * {expert, first sorted position, rows, 0} per m-tile and {-1,0,0,0} past the last one; passing
 * it to qmoe_grouped_qmm saves each workgroup a search of tile_off.
 * Replaces order = argsort(exp), inv = argsort(order) (src/quanta/modeling/moe.py:81-85;
 * src/quanta/dsv4/moe.py:107-112). */
int qmoe_permute(const int32_t* idx, int64_t N, int k, int E, int m_tile, int32_t* counts,
                 int32_t* offsets, int32_t* tile_off, int32_t* sorted_slot, int32_t* inv,
                 int32_t* tile_map, int64_t max_tiles, void* stream);

/* Grouped matmul over expert segments: out[p, :] = act[row(p)] . W_e^T for sorted positions
 * p of expert e (offsets/tile_off from qmoe_permute; m_tile 16 for QMOE_REGIME_SMALL, 128 for
 * QMOE_REGIME_LARGE), with row(p) = slot_of[p] / slot_div (slot_of NULL: row(p) = p). With
 * offsets == NULL the call is one dense segment of dense_rows rows. W is tiled int3/int4/int6
 * (codes + sb), tiled int8 (codes + sb; small regime, K % 64 == 0) or tiled bf16 (codes),
 * [n_experts][n_rows][K]; row_exp (int4; required in the large regime, else ignored) holds
 * the per-row exponents of qmoe_row_exponents for the large regime's fp16 dequant. Epilogue QMOE_EPI_SWIGLU treats
 * rows [0, n_rows/2) as gate and [n_rows/2, n_rows) as up, with the gated activation `glu`
 * (QMOE_ACT_*; glu_alpha and glu_limit as act_alpha and act_limit of qmoe_config_t; other
 * epilogues ignore them).
 * Replaces mx.gather_qmm(..., transpose=True, group_size=64, bits=4)
 * (src/quanta/qwen35/moe.py:117-123, src/quanta/dsv4/moe.py:119-124) with the SwiGLU of
 * src/quanta/qwen35/moe.py:59-63 fused, and mx.gather_mm (src/quanta/qwen35/moe.py:79-81). */
int qmoe_grouped_qmm(const uint16_t* act, int64_t act_rows, const int32_t* slot_of, int slot_div,
                     int64_t n_slots, const int32_t* offsets, const int32_t* tile_off,
                     const int32_t* tile_map, int n_experts, int64_t dense_rows, int K,
                     int n_rows, int weight_format,
                     const void* codes, const uint16_t* sb, const int8_t* row_exp, int epilogue,
                     int glu,
                     float glu_alpha, float glu_limit, void* out, int ld_out,
                     int regime, void* ws, size_t ws_bytes, void* stream);
/* Workspace qmoe_grouped_qmm needs: the large-M int4 regime stages an fp16 copy of the
 * activations (per-row power-of-two scaled, exact for bf16 inputs); otherwise 0. */
size_t qmoe_grouped_qmm_workspace(int64_t act_rows, int K, int weight_format, int regime);

/* y[t] = bf16(sum_s w[t,s] * d[inv[t*k+s]] + shared_gate[t] * shared_out[t]) (fp32 sums in
 * slot order; shared_out/shared_gate may be NULL). Replaces the combine
 * mx.sum(slots.astype(f32) * w[..., None], axis=1) and the final add/cast
 * (src/quanta/qwen35/moe.py:191,201-202; sorted unpermute src/quanta/modeling/moe.py:94-97). */
int qmoe_combine(const uint16_t* d, const int32_t* inv, const float* w, int64_t N, int k, int H,
                 const uint16_t* shared_out, const float* shared_gate, uint16_t* y, void* stream);

/* Bit-exact dequant of a native affine int3, int4, int6 or int8 stack, group 64 or 128:
 * out[rows, in] bf16 = bf16(fma(scale, code, bias)), codes LSB-first (32 per 3 words, 8 per word,
 * 16 per 3 words, 4 per word). Replaces mx.dequantize
 * (src/quanta/bake/quant.py:32-36; src/quanta/qwen35/artifact.py:105-115); int8 g64 is the
 * bake's shared-expert format (src/quanta/qwen35/bake.py:106-110, 143-151). */
int qmoe_dequant(const uint32_t* packed, const uint16_t* scale, const uint16_t* bias, int64_t rows,
                 int64_t in_features, int bits, int group_size, uint16_t* out, void* stream);

/* One-time layout transform of a native int4 stack [n_mats][rows][in] (packed u32 [.., in/8],
 * scale/bias bf16 [.., in/group_size], group_size 64 or 128) into the MFMA-tiled layout
 * (codes: same byte count; sb: [n_mats][rows/16][in/128][16][2][2] bf16, one (scale, bias) per
 * 64 columns: a 128-column group's pair is written for both of its halves, so every kernel
 * reads one layout). rows % 16 == 0, in % 128 == 0. Group 128 is the layout of Kimi's
 * QuantizedSparseMoE stacks (src/quanta/modeling/quantized.py:29-34). Stands in for
 * holding the packed triplet verbatim (Qwen35MoEModule.set_experts_packed,
 * src/quanta/qwen35/model.py:49-55; Qwen35Artifact.moe_packed,
 * src/quanta/qwen35/artifact.py:205-229). */
int qmoe_tile_int4(const uint32_t* packed, const uint16_t* scale, const uint16_t* bias,
                   int64_t n_mats, int64_t rows, int64_t in_features, int group_size,
                   uint32_t* tiled_codes, uint16_t* tiled_sb, void* stream);

/* One-time layout transform of a native int3 stack [n_mats][rows][in] (packed u32 [.., in*3/32],
 * LSB-first bitstream; scale/bias bf16 [.., in/group_size], group 64 or 128) into the tiled int3
 * layout the decode kernel streams: per 16-row tile and 128-deep superblock a 512-byte plane of
 * the codes' low two bits then a 256-byte plane of their top bits (same byte count as the native
 * codes); sb as qmoe_tile_int4. Stands in for holding Kimi's int3 stacks verbatim
 * (QuantizedSparseMoE.set_experts, src/quanta/modeling/quantized.py:38-49). */
int qmoe_tile_int3(const uint32_t* packed, const uint16_t* scale, const uint16_t* bias,
                   int64_t n_mats, int64_t rows, int64_t in_features, int group_size,
                   uint32_t* tiled_codes, uint16_t* tiled_sb, void* stream);

/* One-time layout transform of a native int6 stack [n_mats][rows][in] (packed u32 [.., in*6/32],
 * the bake's LSB-first bitstream, src/quanta/bake/quant.py:48-63; scale/bias bf16
 * [.., in/group_size], group 64 or 128) into the tiled int6 layout the decode kernel streams: per
 * 16-row tile and 128-deep superblock a 1 KiB plane of the codes' low nibbles, laid out as the int4
 * tiles, then a 512-byte plane of their high two bits (same byte count as the native codes); sb as
 * qmoe_tile_int4. Stands in for holding MiniMax M3's int6 triplets verbatim
 * (src/quanta/minimax/model_m3.py:414-450). */
int qmoe_tile_int6(const uint32_t* packed, const uint16_t* scale, const uint16_t* bias,
                   int64_t n_mats, int64_t rows, int64_t in_features, int group_size,
                   uint32_t* tiled_codes, uint16_t* tiled_sb, void* stream);

/* Per weight row of an affine stack [n_mats][rows][in] (native scale/bias bf16
 * [.., in/group_size]): row_exp[r] = 14 - ex, 2^(ex-1) <= M_r < 2^ex, M_r the row's largest
 * dequantized magnitude max_g max(|b_g|, |(2^bits - 1) s_g + b_g|); 0 for an all-zero row; within
 * [-100, 100]. The prefill (large-regime) kernels dequantize int4 weights to fp16 as
 * fp16(2^(row_exp - 20) (s q + b)) (the code nibble enters the fp16 FMA as a subnormal, so the
 * scale is taken times 2^24 or 2^20, which row_exp keeps below fp16's maximum) and undo the
 * power of two on the fp32 result, so rows of any magnitude keep fp16's precision (scales far
 * below fp16's normal range, 2^-14, would otherwise lose bits or vanish). No counterpart in the reference (MLX dequantizes in bf16);
 * computed once per stack with the tiling. */
int qmoe_row_exponents(const uint16_t* scale, const uint16_t* bias, int64_t n_mats, int64_t rows,
                       int64_t in_features, int bits, int group_size, int8_t* row_exp,
                       void* stream);

/* One-time layout transform of a native int8 matrix stack [n_mats][rows][in] (packed u32
 * [.., in/4], code k in byte k%4 of word k/4; scale/bias bf16 [.., in/group_size], group 64 or
 * 128) into the tiled int8 layout: codes [n_mats][rows/16][in/32][64 lanes][8 codes] (lane l:
 * row l%16, codes 32c + 8(l/16) .. +8, the bf16 tiling at one byte per weight) and sb
 * [n_mats][rows/16][in/64][16 rows][scale, bias] bf16 (a 128-column group's pair written for
 * both of its halves). rows % 16 == 0, in % 64 == 0. Stands in for the load-time dequant of the
 * bake's int8 shared expert (src/quanta/qwen35/artifact.py:171-184): the kernels read the codes
 * and dequantize in registers. */
int qmoe_tile_int8(const uint32_t* packed, const uint16_t* scale, const uint16_t* bias,
                   int64_t n_mats, int64_t rows, int64_t in_features, int group_size,
                   uint32_t* tiled_codes, uint16_t* tiled_sb, void* stream);

/* Inverse check of qmoe_tile_int4: tiled stack -> bf16 [n_mats][rows][in], bit-identical to
 * qmoe_dequant of the native stack. Test/inspection entry point. */
int qmoe_dequant_tiled(const uint32_t* tiled_codes, const uint16_t* tiled_sb, int64_t n_mats,
                       int64_t rows, int64_t in_features, uint16_t* out, void* stream);

/* Row-major bf16 [n_mats][rows][in] -> MFMA-tiled [n_mats][rows/16][in/32][64][8].
 * rows % 16 == 0, in % 32 == 0. Used for the shared expert, the bf16 router and bf16
 * routed experts (set_experts, src/quanta/qwen35/model.py:46-47). */
int qmoe_tile_bf16(const uint16_t* w, int64_t n_mats, int64_t rows, int64_t in_features,
                   uint16_t* tiled, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* QUANTA_MOE_H_ */
