/*
 * janus_moe.h - C ABI of the MI355X (gfx950) W4A16 mixture-of-experts layer.
 *
 * Every entry point takes plain device pointers, sizes and a hipStream_t, launches its kernels on that stream
 * and returns at once: no allocation, no host synchronisation, no device-to-host read. Scratch memory comes from
 * the caller through `ws` / `ws_bytes` (ask the matching *_workspace_bytes function for the size). The calls are
 * re-entrant; the process state is a thread-local error string and one status word per device that kernels set
 * when something goes wrong on the device (janus_moe_device_status). Return value 0 is success; any other value
 * is an error code below, with a message in janus_moe_last_error().
 *
 * Tensor conventions (row-major, innermost dimension last, no padding):
 *   bf16 values travel as uint16_t bit patterns.
 *   int4 weights: int32 words [rows, K/8]; element k = 8*j + i of a row lives in bits 4i..4i+3 of word j, two's
 *   complement in [-8, 7]. Scales: bf16 [rows, K/128], one per 128 consecutive k. The weight value is
 *   bf16(float(q) * float(scale)), rounded to nearest even once.
 *   Expert stacks: gate_up words [E, 2I, H/8] (rows 0..I-1 gate, I..2I-1 up), scales [E, 2I, H/128];
 *   down words [E, H, I/8], scales [E, H, I/128].
 *   NVFP4 weights (the ModelOpt layout janus/hybrid.py loads): e2m1 codes packed two per byte [rows, K/2] uint8
 *   (low nibble = even k; bit 3 sign, bits 2-1 exponent, bit 0 mantissa), OCP e4m3 block scales [rows, K/16] uint8,
 *   an fp32 global scale per row [rows]. The weight value is bf16(fp32(e2m1 * fp32(scale * global))): two fp32
 *   products, then one rounding to bf16, as the reference's dequantise path and fused kernel compute it.
 */
#ifndef JANUS_MOE_H
#define JANUS_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__)
#define JANUS_MOE_API __attribute__((visibility("default")))
#else
#define JANUS_MOE_API
#endif

typedef struct ihipStream_t* janus_stream_t; /* the same handle type as hipStream_t */

enum {
  JANUS_MOE_OK = 0,
  JANUS_MOE_EINVAL = 1,     /* a size, shape or pointer argument is not supported */
  JANUS_MOE_EWORKSPACE = 2, /* ws_bytes is smaller than the matching *_workspace_bytes() */
  JANUS_MOE_ELAUNCH = 3     /* the HIP runtime refused a launch */
};

/* Message of the last failing call on this thread ("" when none). */
JANUS_MOE_API const char* janus_moe_last_error(void);
/* Bumped whenever a signature below changes. */
JANUS_MOE_API int janus_moe_abi_version(void);

/* Profiling hook with no counterpart in the reference: while set (count > 0), the experts and block pipelines of the
 * calling thread record events[i] (hipEvent_t) on their stream at stage boundaries: 0 start, 1 before align,
 * 2 before the gate_up GEMM, 3 before the down GEMM, 4 before the combine, 5 end. count = 0 turns it off. The events
 * belong to the caller; at most 6. */
JANUS_MOE_API int janus_moe_profile_events(void* const* events, int count);

/* Sticky status of this library's kernels on the calling thread's current device. No counterpart in the reference,
 * whose torch ops fail inside the call; these kernels run asynchronously and report here instead. Bits:
 *   1  a down unit of the persistent experts launch gave up waiting for the h rows it reads (after
 *      JANUS_MOE_SPIN_LIMIT polls of about 1 us, default 2^18, read at each launch; 0 gives up at once): the output
 *      rows of that unit's tokens are NaN, never a silently wrong value;
 *   2  an expert id outside [0, E) reached janus_moe_experts, janus_moe_experts_nvfp4 or janus_moe_align: that
 *      assignment was dropped (it contributes nothing; the reference's index_add_ would have raised).
 * Copies the word (every bit set on this device since it was last cleared) into out, device memory holding one
 * int32, on the stream, then clears it when clear != 0. Read out after synchronising the stream. */
JANUS_MOE_API int janus_moe_device_status(int32_t* out, int clear, janus_stream_t stream);

/* ------------------------------------------------------------------------------------------------------------
 * Router.
 * janus_moe_router_prepare has no counterpart in the reference: it splits the fp32 router weight [E, H] once
 * into two bf16 planes plus the norms the selection uses (a layout transform of a fixed weight, done at load
 * time). `prep` is device memory of janus_moe_router_prep_bytes(E, H) bytes.
 */
JANUS_MOE_API size_t janus_moe_router_prep_bytes(int E, int H);
JANUS_MOE_API int janus_moe_router_prepare(const float* w_router, int E, int H, void* prep, size_t prep_bytes,
                             janus_stream_t stream);

/* Replaces Qwen3_5MoeTopKRouter.forward (transformers models/qwen3_5_moe/modeling_qwen3_5_moe.py:768-776)
 * plus the shared-expert gate sigmoid (same file :794).
 *   x [T, H] bf16, w_router [E, H] fp32, prep from janus_moe_router_prepare, bias [E] fp32 or NULL (added to
 *   the logits), w_shared_gate [H] bf16 or NULL.
 *   Outputs: topk_idx [T, top_k] int32 (slot order: logit descending, ties to the lower expert id),
 *   topk_w [T, top_k] fp32 (softmax over the logits renormalised over the top_k), gamma [T] fp32 =
 *   sigmoid(x . w_shared_gate) (ignored when w_shared_gate is NULL).
 *   Logit of (t, e): the fp32 rounding (nearest even) of the exact dot product x[t] . w_router[e], plus bias[e]
 *   in fp32. Selection and slot order are bit-exact under that rule. */
JANUS_MOE_API size_t janus_moe_route_workspace_bytes(int T, int H, int E);
JANUS_MOE_API int janus_moe_route(const uint16_t* x, const float* w_router, const void* prep, const float* bias,
                    const uint16_t* w_shared_gate, int T, int H, int E, int top_k, int32_t* topk_idx,
                    float* topk_w, float* gamma, void* ws, size_t ws_bytes, janus_stream_t stream);

/* ------------------------------------------------------------------------------------------------------------
 * Replaces align(top_k_index, num_experts, block) (janus/moe_w4a16.py:89-106), bit-exact:
 *   top_k_index [S, top_k] int64 with values in [0, E);
 *   sorted_ids [tiles * block] int64, expert_ids [tiles] int64, total [1] int64, where
 *   tiles = (S*top_k + E*(block-1) + block - 1) / block. Assignment ids sorted stably by expert, each expert
 *   padded to a multiple of `block` with the sentinel S*top_k; expert_ids[i] = the expert owning rows
 *   [i*block, (i+1)*block), E or more past `total`; total = the padded row count. */
JANUS_MOE_API size_t janus_moe_align_workspace_bytes(int S, int top_k, int E);
JANUS_MOE_API int janus_moe_align(const int64_t* top_k_index, int S, int top_k, int E, int block, int64_t* sorted_ids,
                    int64_t* expert_ids, int64_t* total, void* ws, size_t ws_bytes, janus_stream_t stream);

/* ------------------------------------------------------------------------------------------------------------
 * Replaces fused_moe(x, top_k_index, top_k_weights, gate_up, ..., down, ...) (janus/moe_w4a16.py:122-140) and
 * NVFP4Experts.forward (janus/hybrid.py:551-572) for the int4 group-128 codec:
 *   out[s] = bf16( sum_j top_k_weights[s, j] * down_e( bf16(silu(gate_e(x[s])) * up_e(x[s])) ) ), e =
 *   top_k_index[s, j]; every dot product accumulates in fp32; each weighted term is held as int16 codes with one
 *   fp32 scale per 64 columns (error at most 2^-16 of the block's largest |term|), and the sum over j is fp32,
 *   rounded once.
 *   x [S, H] bf16, top_k_index [S, top_k] int64, top_k_weights [S, top_k] fp32, out [S, H] bf16.
 *   Requires H % 128 == 0 and I % 128 == 0, and below 2 GiB: S*H and (S*top_k + 15*E)*I bf16 values.
 *   Ids must lie in [0, E): one outside is dropped (its term is left out of the sum) and reported as status bit 2
 *   (janus_moe_device_status). */
JANUS_MOE_API size_t janus_moe_experts_workspace_bytes(int S, int top_k, int E, int H, int I);
JANUS_MOE_API int janus_moe_experts(const uint16_t* x, const int64_t* top_k_index, const float* top_k_weights,
                      const int32_t* gate_up_q, const uint16_t* gate_up_s, const int32_t* down_q,
                      const uint16_t* down_s, int S, int H, int I, int E, int top_k, uint16_t* out, void* ws,
                      size_t ws_bytes, janus_stream_t stream);

/* ------------------------------------------------------------------------------------------------------------
 * Replaces fused_moe (janus/moe_w4a16.py:122-140) on its own NVFP4 stacks, the reference's arguments one for one:
 *   gate_up [E, 2I, H/2] uint8, gate_up_scale [E, 2I, H/16] e4m3 bytes, gate_up_global [E, 2I] fp32 (the reference's
 *   [E, 2I, 1]), down [E, H, I/2], down_scale [E, H, I/16], down_global [E, H]. Same outputs and numerics as
 *   janus_moe_experts apart from the decode; same workspace (janus_moe_experts_workspace_bytes). */
JANUS_MOE_API int janus_moe_experts_nvfp4(const uint16_t* x, const int64_t* top_k_index, const float* top_k_weights,
                                          const uint8_t* gate_up, const uint8_t* gate_up_scale,
                                          const float* gate_up_global, const uint8_t* down, const uint8_t* down_scale,
                                          const float* down_global, int S, int H, int I, int E, int top_k,
                                          uint16_t* out, void* ws, size_t ws_bytes, janus_stream_t stream);

/* ------------------------------------------------------------------------------------------------------------
 * fused_moe with a reused tile plan (janus/moe_w4a16.py:122-140, `plan=`; the plan comes from align() at :129-130):
 * plan_sorted_ids [tiles * block] and plan_expert_ids [tiles] int64, tiles = ceil((S*top_k + E*(block-1)) / block),
 * as janus_moe_align(top_k_index, E, block) writes them for this top_k_index. The align launch is skipped; the
 * GEMMs take their row order from the plan (the same rows in the same order per expert, so the output is bit for bit
 * that of janus_moe_experts / janus_moe_experts_nvfp4). codec 0: int4 (gate_up = int32 words, scales bf16, globals
 * NULL), 1: NVFP4 (as janus_moe_experts_nvfp4). A plan for another top_k_index gives a wrong result, but every
 * access stays in bounds. */
JANUS_MOE_API size_t janus_moe_experts_planned_workspace_bytes(int S, int top_k, int E, int H, int I, int block);
JANUS_MOE_API int janus_moe_experts_planned(int codec, const uint16_t* x, const int64_t* top_k_index,
                                            const float* top_k_weights, const void* gate_up, const void* gate_up_scale,
                                            const float* gate_up_global, const void* down, const void* down_scale,
                                            const float* down_global, const int64_t* plan_sorted_ids,
                                            const int64_t* plan_expert_ids, int block, int S, int H, int I, int E,
                                            int top_k, uint16_t* out, void* ws, size_t ws_bytes,
                                            janus_stream_t stream);

/* ------------------------------------------------------------------------------------------------------------
 * Replaces nvfp4_dequantize (janus/hybrid.py:426-437) and with it NVFP4Experts.gate_up_proj / down_proj
 * (:539-545): out [rows, K] bf16 from packed [rows, K/2] uint8, scale [rows, K/16] e4m3 bytes, global [rows] fp32,
 * by the device decode the GEMMs use. K % 16 == 0; stacks [E, N, K] are rows = E * N. */
JANUS_MOE_API int janus_moe_dequant_nvfp4(const uint8_t* packed, const uint8_t* scale, const float* global, long rows,
                                          int K, uint16_t* out, janus_stream_t stream);

/* ------------------------------------------------------------------------------------------------------------
 * Replaces the dequantising properties NVFP4Experts.gate_up_proj / down_proj and NVFP4Linear.weight
 * (janus/hybrid.py:539-545, 502-504) for the int4 codec: out [rows, K] bf16 = bf16(q * s), computed by the same
 * device decode the GEMMs use. q [rows, K/8] int32, s [rows, K/128] bf16; K % 128 == 0. Stacks [E, N, K] are
 * rows = E * N. */
JANUS_MOE_API int janus_moe_dequant(const int32_t* q, const uint16_t* s, long rows, int K, uint16_t* out,
                                    janus_stream_t stream);

/* ------------------------------------------------------------------------------------------------------------
 * Replaces Qwen3_5MoeSparseMoeBlock.forward (transformers models/qwen3_5_moe/modeling_qwen3_5_moe.py:787-798)
 * with int4 expert and shared-expert weights: router, routed experts, shared expert scaled by
 * sigmoid(x . shared_gate), all summed in fp32 and rounded to bf16 once (each term held as in janus_moe_experts). */
typedef struct janus_moe_block_weights {
  int H, I, E, top_k;             /* hidden, routed intermediate, experts, experts per token */
  int I_s;                        /* shared-expert intermediate; 0 = no shared expert */
  const float* router_w;          /* [E, H] fp32 */
  const void* router_prep;        /* janus_moe_router_prepare(router_w) */
  const float* router_bias;       /* [E] fp32 or NULL */
  const int32_t* gate_up_q;       /* [E, 2I, H/8] */
  const uint16_t* gate_up_s;      /* [E, 2I, H/128] */
  const int32_t* down_q;          /* [E, H, I/8] */
  const uint16_t* down_s;         /* [E, H, I/128] */
  const int32_t* sh_gate_up_q;    /* [2 I_s, H/8] */
  const uint16_t* sh_gate_up_s;   /* [2 I_s, H/128] */
  const int32_t* sh_down_q;       /* [H, I_s/8] */
  const uint16_t* sh_down_s;      /* [H, I_s/128] */
  const uint16_t* sh_gate_w;      /* [H] bf16 (shared_expert_gate.weight) */
} janus_moe_block_weights;

/* topk_idx / topk_w: optional [T, top_k] copies of the routing (NULL to skip). */
JANUS_MOE_API size_t janus_moe_block_workspace_bytes(int T, int H, int I, int E, int top_k, int I_s);
JANUS_MOE_API int janus_moe_block_forward(const janus_moe_block_weights* w, const uint16_t* x, int T, uint16_t* out,
                            int32_t* topk_idx, float* topk_w, void* ws, size_t ws_bytes, janus_stream_t stream);

/* ------------------------------------------------------------------------------------------------------------
 * janus_moe_block_forward over a level batch with right padding: the caller's `valid` mask (janus/hybrid.py:
 * 1730-1745 builds it per level, [rows, length] bool, False = padding) flattened to [T] bytes, nonzero = a real
 * token. Padding tokens are routed to no expert (topk_idx = E, topk_w = 0), so the expert GEMMs skip their rows, and
 * their output rows are zero; real tokens get bit for bit the unmasked result. valid NULL = every token. Device
 * memory, read on the stream, so a captured graph replays with whatever mask the buffer holds. */
JANUS_MOE_API int janus_moe_block_forward_masked(const janus_moe_block_weights* w, const uint16_t* x,
                                                 const uint8_t* valid, int T, uint16_t* out, int32_t* topk_idx,
                                                 float* topk_w, void* ws, size_t ws_bytes, janus_stream_t stream);

/* ------------------------------------------------------------------------------------------------------------
 * The same block with the checkpoint's own NVFP4 weights, the layer load_nvfp4 builds (janus/hybrid.py:1462-1475):
 * routed experts as NVFP4Experts stacks (janus/hybrid.py:512-572) and the shared expert's gate_proj / up_proj /
 * down_proj as NVFP4Linear (:483-509), decoded inside the GEMMs as janus_moe_experts_nvfp4 does; router, shared gate,
 * valid mask, outputs and workspace (janus_moe_block_workspace_bytes) as in janus_moe_block_forward_masked. The
 * shared expert's gate and up weights are stacked like the routed ones (gate rows first), each row with its own fp32
 * global scale (a linear's weight_scale_2 repeated over its rows). */
typedef struct janus_moe_block_weights_nvfp4 {
  int H, I, E, top_k;             /* hidden, routed intermediate, experts, experts per token */
  int I_s;                        /* shared-expert intermediate; 0 = no shared expert */
  const float* router_w;          /* [E, H] fp32 */
  const void* router_prep;        /* janus_moe_router_prepare(router_w) */
  const float* router_bias;       /* [E] fp32 or NULL */
  const uint8_t* gate_up;         /* [E, 2I, H/2] e2m1 pairs */
  const uint8_t* gate_up_scale;   /* [E, 2I, H/16] e4m3 */
  const float* gate_up_global;    /* [E, 2I] fp32 */
  const uint8_t* down;            /* [E, H, I/2] */
  const uint8_t* down_scale;      /* [E, H, I/16] */
  const float* down_global;       /* [E, H] */
  const uint8_t* sh_gate_up;      /* [2 I_s, H/2] */
  const uint8_t* sh_gate_up_scale;/* [2 I_s, H/16] */
  const float* sh_gate_up_global; /* [2 I_s] */
  const uint8_t* sh_down;         /* [H, I_s/2] */
  const uint8_t* sh_down_scale;   /* [H, I_s/16] */
  const float* sh_down_global;    /* [H] */
  const uint16_t* sh_gate_w;      /* [H] bf16 (shared_expert_gate.weight) */
} janus_moe_block_weights_nvfp4;

JANUS_MOE_API int janus_moe_block_forward_nvfp4(const janus_moe_block_weights_nvfp4* w, const uint16_t* x,
                                                const uint8_t* valid, int T, uint16_t* out, int32_t* topk_idx,
                                                float* topk_w, void* ws, size_t ws_bytes, janus_stream_t stream);

/* ------------------------------------------------------------------------------------------------------------
 * janus_moe_block_forward_masked without a workspace argument. No counterpart in the reference: it is for callers
 * that cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). Its scratch is a static device array of JANUS_MOE_NOALLOC_SCRATCH_BYTES per GPU (64 MiB, held until
 * the process ends); a call whose janus_moe_block_workspace_bytes exceeds it returns JANUS_MOE_EWORKSPACE (at the
 * 35B-A3B shape, H 2048, 256 experts top-8, I = I_s = 512, that is above 1,134 tokens). Nothing is allocated.
 * Every call on one GPU uses that GPU's array and leaves its contents behind (each call writes what it reads first),
 * so calls that overlap in time on one GPU, from several streams or threads, race. Same outputs, bit for bit, as
 * janus_moe_block_forward_masked. */
#define JANUS_MOE_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
JANUS_MOE_API int janus_moe_block_forward_noalloc(const janus_moe_block_weights* w, const uint16_t* x,
                                                  const uint8_t* valid, int T, uint16_t* out, int32_t* topk_idx,
                                                  float* topk_w, janus_stream_t stream);

/* ------------------------------------------------------------------------------------------------------------
 * Replaces _add_norm (janus/hybrid.py:267-273, with _rmsnorm :250-254): x_out = residual + h in bf16 (torch's bf16 add:
 * the fp32 sum rounded once; h NULL = no add) and n_out = Qwen3_5RMSNorm(x_out) =
 * bf16(fp32(x) * rsqrt(mean(fp32(x)^2) + eps) * (1 + fp32(weight))), zeroed where valid[t] == 0 (valid NULL: no mask).
 * [T, H] bf16 rows, weight [H] bf16; H % 4 == 0, H <= 4096. x_out may be NULL or alias residual; n_out may alias h. */
JANUS_MOE_API int janus_moe_add_rmsnorm(const uint16_t* residual, const uint16_t* h, const uint16_t* weight, float eps,
                                        const uint8_t* valid, int T, int H, uint16_t* x_out, uint16_t* n_out,
                                        janus_stream_t stream);

/* ------------------------------------------------------------------------------------------------------------
 * The MoE layer with its serving neighbours (janus/hybrid.py:1096-1105, `_serve_level`): the post-attention
 * _add_norm, the block, and the next _add_norm with the block's output as its h, which replaces
 *   x1, n1 = _add_norm(x, h_attn, post_norm_w, post_eps, None);  moe = block(n1);
 *   x_out, h_out = _add_norm(x1, moe, next_norm_w, next_eps, next_valid)
 * with the combine writing the second _add_norm directly (the MoE output is never stored). valid (NULL: none) skips
 * padding tokens in the block as janus_moe_block_forward_masked does (their moe is 0). x_out may alias x; h_out must
 * alias neither; h_attn may alias h_out. Workspace: janus_moe_block_workspace_bytes. */
JANUS_MOE_API int janus_moe_block_forward_serve(const janus_moe_block_weights* w, const uint16_t* x,
                                                const uint16_t* h_attn, const uint16_t* post_norm_w, float post_eps,
                                                const uint16_t* next_norm_w, float next_eps, const uint8_t* valid,
                                                const uint8_t* next_valid, int T, uint16_t* x_out, uint16_t* h_out,
                                                int32_t* topk_idx, float* topk_w, void* ws, size_t ws_bytes,
                                                janus_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* JANUS_MOE_H */
