/*
 * tinyserve_amd — C ABI of the MI355X (gfx950) expert-FFN library.
 *
 * Conventions (every entry point):
 *   - pointers named w / data / blocks / scales / x / y / slots / weights / logits /
 *     pool / workspace are DEVICE pointers; sizes are int64_t element or byte counts;
 *   - `stream` is a hipStream_t passed as void* (NULL = the null stream); work is
 *     enqueued asynchronously on it and nothing is synchronised;
 *   - the library allocates nothing per call and keeps no pointer after return;
 *     outputs and workspaces are caller-allocated;
 *   - return value: 0 (TSA_OK) or a negative tsa_status; tsa_last_error() then
 *     holds a message for the calling thread.
 *
 * ggml type ids: 8 = Q8_0, 12 = Q4_K, 13 = Q5_K, 14 = Q6_K (0 = F32, 1 = F16 for dequant).
 * GGUF matrices use ggml's (ne0 = in = K, ne1 = out = N) convention: element (n, k)
 * is flat index n*K + k of the block stream, so rows may straddle 256-value blocks.
 */
#ifndef TINYSERVE_AMD_H
#define TINYSERVE_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum tsa_status {
    TSA_OK = 0,
    TSA_ERR_INVALID_ARG = -1,
    TSA_ERR_UNSUPPORTED_TYPE = -2,
    TSA_ERR_SHAPE = -3,
    TSA_ERR_WEIGHT_TOO_SMALL = -4,
    TSA_ERR_ACT_TOO_SMALL = -5,
    TSA_ERR_WORKSPACE = -6,
    TSA_ERR_HIP = -7
} tsa_status;

typedef enum tsa_dtype { TSA_F32 = 0, TSA_F16 = 1, TSA_BF16 = 2 } tsa_dtype;

typedef enum tsa_route_mode {
    TSA_ROUTE_TOPK_SOFTMAX = 0,        /* topk(logits) then softmax over the k values (GPT-OSS) */
    TSA_ROUTE_SOFTMAX_TOPK = 1,        /* softmax(logits) then topk, no renormalisation        */
    TSA_ROUTE_SOFTMAX_TOPK_RENORM = 2  /* softmax -> topk -> divide by the k-sum (Qwen3-MoE)   */
} tsa_route_mode;

typedef enum tsa_act { TSA_ACT_SILU = 0, TSA_ACT_SWIGLU_OAI = 1 } tsa_act;

typedef enum tsa_expert_format { TSA_EXPERT_MXFP4 = 1, TSA_EXPERT_GGUF = 2 } tsa_expert_format;

/* Where one expert's tensors sit inside a packed slot (byte offsets from the slot start).
 *  MXFP4 (GPT-OSS): gate_up blocks [2I, H/32, 16] u8 at gate_off (rows interleaved:
 *    even = gate, odd = up), gate_up scales [2I, H/32] u8 at gate_scales_off,
 *    down blocks [H, I/32, 16] at down_off, down scales [H, I/32] at down_scales_off,
 *    optional biases [2I] / [H] of bias_dtype at gate_bias_off / down_bias_off (-1 = none).
 *    mx_tiled = 1: both matrices are instead stored in the 16-row MFMA tile order that
 *    tsa_mxfp4_tile produces (the fast decode path); 0: the checkpoint order above.
 *  GGUF: gate [I x H] of gate_type at gate_off, up [I x H] of up_type at up_off,
 *    down [H x I] of down_type at down_off (GGUF has no biases; set them to -1).
 *  act: TSA_ACT_SWIGLU_OAI = (up+1)*g*sigmoid(alpha*g), g = min(gate, limit),
 *    up = clamp(up, -limit, limit); TSA_ACT_SILU = silu(gate)*up.
 *  prefill_mfma (tiled MXFP4 prefill GEMMs): TSA_PREFILL_FP6 (0, the default) multiplies the
 *    fp4 weights with activations carried as two fp6 (e2m3) terms per value with
 *    per-32-block scales, on the scaled MFMA (v_mfma_scale_f32_32x32x64_f8f6f4);
 *    TSA_PREFILL_BF16 (1) expands the weights to bf16 for v_mfma_f32_32x32x16_bf16. */
typedef struct tsa_expert_layout {
    int32_t format;
    int32_t act;
    int64_t hidden;
    int64_t inter;
    int64_t slot_bytes;
    int32_t gate_type, up_type, down_type, bias_dtype;
    int64_t gate_off, up_off, down_off;
    int64_t gate_scales_off, down_scales_off;
    int64_t gate_bias_off, down_bias_off;
    float swiglu_limit, swiglu_alpha;
    int32_t mx_tiled;
    int32_t prefill_mfma;
} tsa_expert_layout;

typedef enum tsa_prefill_mfma { TSA_PREFILL_FP6 = 0, TSA_PREFILL_BF16 = 1 } tsa_prefill_mfma;

/* ---- library info / errors (no reference counterpart) ---- */
int tsa_version(void);
const char* tsa_status_string(int status);
const char* tsa_last_error(void);

/* Block geometry of a ggml type: values per block and bytes per block.
 * Replaces the GGML_TYPES table lookups (tinyserve/gguf_reader.py:15-29). */
int tsa_gguf_block_info(int ggml_type, int64_t* block_elems, int64_t* type_size);

/* Bit-exact GGUF dequantisation of n_elems values (a whole number of blocks) into
 * out (out_dtype F32, or BF16/F16 rounded to nearest even).
 * Replaces dequant_tensor (tinyserve/gguf_dequant_torch.py:35-78). */
int tsa_gguf_dequant(int ggml_type, const void* data, int64_t data_bytes, int64_t n_elems,
                     void* out, int out_dtype, void* stream);

/* y[t, n] = sum_k W[n, k] * x[t, k] for t < T, with W an N x K GGUF matrix.
 * Requires K % 32 == 0 and N*K a whole number of blocks; x has T*K elements.
 * Replaces torch.ops.tinyserve_ggml.ggml_mul_mat_vec (tinyserve/csrc/ggml_ops.cu:461-569)
 * and the per-token loop of GGMLLinear.forward (tinyserve/ggml_linear.py:86-100). */
int tsa_gguf_matvec(int ggml_type, const void* w, int64_t w_bytes,
                    const void* x, int x_dtype, int64_t T, int64_t K,
                    void* y, int y_dtype, int64_t N, void* stream);

/* Bit-exact MXFP4 dequantisation to [N, K] (transpose = 0) or [K, N] (transpose = 1).
 * Replaces dequant_mxfp4_no_transpose / dequant_mxfp4 (tinyserve/mxfp4.py:20-53). */
int tsa_mxfp4_dequant(const void* blocks, const void* scales, int64_t N, int64_t K,
                      void* out, int out_dtype, int transpose, void* stream);

/* Sizes of an MXFP4 matrix [N, K] (N % 16 == 0, K % 32 == 0) in the 16-row MFMA tile
 * order: blocks_bytes = N*K/2 (same as the checkpoint order), scales_bytes = N/16 *
 * 256 * ceil(ceil(K/128)/4) (per-lane scale words, zero-padded).
 * No reference counterpart: the tile order is this library's device layout. */
int tsa_mxfp4_tile_sizes(int64_t N, int64_t K, int64_t* blocks_bytes, int64_t* scales_bytes);

/* Repack an MXFP4 matrix from the checkpoint order (blocks [N, K/32, 16], scales
 * [N, K/32]) into the 16-row MFMA tile order: tile r = rows 16r..16r+15 is 8*K
 * contiguous bytes whose 1 KB piece m holds, at 16*(16*q + i), the 16-byte block 4m+q
 * of row 16r+i (a wave's 16-byte-per-lane load of piece m is one MFMA operand); the
 * scale of that block is byte m%4 of 32-bit word m/4 of lane 16q+i, each lane's words
 * stored in lane-major chunks of up to 4 words (see mx_tile.hip). Out-of-place; the caller owns both outputs. Used when experts are
 * copied into the resident pool (the reference copies the checkpoint bytes as they are:
 * ExpertStore.copy_to_buffer_slot / copy_to_buffer, tinyserve/expert_store.py:532-560). */
int tsa_mxfp4_tile(const void* blocks, const void* scales, int64_t N, int64_t K,
                   void* tiled_blocks, void* tiled_scales, void* stream);

/* y[t, n] = sum_k deq(W)[n, k] * x[t, k] + bias[n] (bias may be NULL).
 * Replaces dot_scaled_vecmat (tinyserve/triton_dot_scaled.py:68-122) /
 * fused_dequant_vecmat (tinyserve/triton_dequant.py:105-139) / _mxfp4_linear
 * (tinyserve/_model_hooks.py:105-116). */
int tsa_mxfp4_matvec(const void* blocks, const void* scales, const void* bias, int bias_dtype,
                     const void* x, int x_dtype, int64_t T,
                     void* y, int y_dtype, int64_t N, int64_t K, void* stream);

/* Router top-k over logits [T, E] (logits_dtype F32/BF16/F16): idx [T, k] int32 and
 * weights [T, k] f32, descending, ties to the lower expert id.
 * Replaces the route closures of _extract_routing_fn (tinyserve/_model_hooks.py:424-476). */
int tsa_route_topk(const void* logits, int logits_dtype, int64_t T, int64_t E, int k, int mode,
                   int32_t* idx, float* weights, void* stream);

/* Router logits of the MoE block's linear gate: out [T, E] = x [T, H] . w [E, H]^T (+ bias [E],
 * optional), fp32 accumulation and one rounding to out_dtype, as the router nn.Linear
 * computes them (bf16 for GPT-OSS). H a multiple of 8; x and w 16-byte aligned (32 for
 * f32). Feeds tsa_route_topk / tsa_moe_decode_routed on the device: replaces the router
 * call ahead of the routing closures (tinyserve/_model_hooks.py:424-476; GPT-OSS router
 * with bias :441-444). */
int tsa_router_logits(const void* x, int x_dtype, int64_t T, int64_t H, const void* w, int w_dtype,
                      const void* bias, int bias_dtype, int64_t E, void* out, int out_dtype, void* stream);

/* Workspace bytes tsa_moe_decode needs for T tokens with top-k experts. The workspace
 * starts with a 32 KiB sync area, the only part that carries state from one call to the
 * next (the one-launch MXFP4 decode's call counter and workgroup flags): before the first
 * call on a workspace every 32-bit word of it must hold one value (zero the workspace, or
 * fill it with any one byte); the library keeps it consistent after that. */
int tsa_moe_decode_workspace_size(const tsa_expert_layout* layout, int64_t T, int k, int64_t* bytes);

/* Fused top-k expert FFN over resident packed slots:
 *   y[t] = sum_j weights[t, j] * FFN(pool + slots[t, j] * slot_bytes, x[t]),
 * skipping slots < 0 (they contribute zero). slots [T, k] int32 and weights [T, k] f32
 * stay on the device (no host sync). y is overwritten. The workspace
 * (tsa_moe_decode_workspace_size bytes) needs its sync area cleared once before the first
 * call (see there). Calls that share a workspace must be ordered (one stream).
 * Replaces fast_expert_forward (tinyserve/csrc/expert_loop.cpp:41-123) and the per-expert
 * loops of ExpertPipeline._execute_layer_experts_native / _forward_cache_hits
 * (tinyserve/expert_pipeline.py:241-285,416-496) over GGMLExpertForward
 * (tinyserve/ggml_forward.py:88-115) and the MXFP4 inline forward
 * (tinyserve/expert_forward.py:197-246, tinyserve/_model_hooks.py:376-394). */
int tsa_moe_decode(const tsa_expert_layout* layout, const void* pool, int64_t n_slots,
                   const int32_t* slots, const float* weights, int64_t T, int k,
                   const void* x, int x_dtype, void* y, int y_dtype,
                   void* workspace, int64_t workspace_bytes, void* stream);

/* Router + fused top-k expert FFN in one call: routes logits [T, E] (mode as in
 * tsa_route_topk), maps expert ids to slots through expert_slot [E] (-1: not resident,
 * contributes zero) and computes y as tsa_moe_decode does. idx_out [T, k] / w_out [T, k]
 * (optional, may be NULL) receive the routing. For MXFP4 experts with T <= 4 and E <= 256
 * this is two kernel launches (routing inside both) with no host sync.
 * Replaces the route closure + execute_layer_experts pair of the MoE hook
 * (tinyserve/_model_hooks.py:524-564, tinyserve/expert_pipeline.py:140-164). */
int tsa_moe_decode_routed(const tsa_expert_layout* layout, const void* pool, int64_t n_slots,
                          const int32_t* expert_slot, int64_t E, const void* logits, int logits_dtype, int mode,
                          int64_t T, int k, const void* x, int x_dtype, void* y, int y_dtype,
                          int32_t* idx_out, float* w_out, void* workspace, int64_t workspace_bytes, void* stream);

/* tsa_moe_decode_routed without the workspace argument: it allocates nothing (no hipMalloc,
 * no allocating library call) and works in a device array of 8 MiB per GPU that the library
 * holds until the process ends; calls whose workspace would exceed it (see
 * tsa_moe_decode_workspace_size) return TSA_ERR_WORKSPACE. All calls on one GPU share that
 * array, so calls that overlap on one GPU race: order them on one stream. The tiled MXFP4
 * decode always runs as two launches here (tsa_set_decode_options does not apply), so the
 * array's sync area is never used.
 * No counterpart in the reference. For callers that cannot allocate: code under HIP graph
 * capture, tight serving loops, harnesses that forbid allocation. */
int tsa_moe_decode_routed_noalloc(const tsa_expert_layout* layout, const void* pool, int64_t n_slots,
                                  const int32_t* expert_slot, int64_t E, const void* logits, int logits_dtype,
                                  int mode, int64_t T, int k, const void* x, int x_dtype, void* y, int y_dtype,
                                  int32_t* idx_out, float* w_out, void* stream);

/* Process-wide options of the tiled MXFP4 decode. tiled_form 1 (the default): two launches
 * ordered by the stream; 0: one launch (top-k <= 4, inter a multiple of 64), whose down
 * workgroups wait (bounded) for the gate_up workgroups of their token. wait_limit: polls a
 * one-launch wait makes before it gives up (default 262144, about a quarter second; 0 gives
 * up at once, for tests of the failure path). A wait that gives up writes NaN for the outputs
 * of its workgroup and poisons the workspace's sync area: later calls on it write NaN until
 * it is cleared.
 * No counterpart in the reference (its decode is one host loop over experts). */
int tsa_set_decode_options(int tiled_form, uint32_t wait_limit);

/* Whether a decode workspace is poisoned (a one-launch wait gave up): copies its call
 * counter to the host, synchronising the stream. Clearing the workspace's sync area (see
 * tsa_moe_decode_workspace_size) heals it. No counterpart in the reference. */
int tsa_moe_decode_workspace_status(const void* workspace, int64_t workspace_bytes, int* poisoned, void* stream);

/* Expert-major grouping of the (token, j) assignments idx [T, k] (int32 expert ids in
 * [0, E), ids < 0 ignored): counts [E], offsets [E+1] (exclusive scan), perm [T*k]
 * holding t*k + j, token-major within each expert.
 * Replaces group_tokens_by_expert (tinyserve/_fast_cache.pyx:60-85) and the dict
 * grouping of ExpertPipeline.execute_layer_experts_batched (tinyserve/expert_pipeline.py:187-200). */
int tsa_group_by_expert(const int32_t* idx, int64_t T, int k, int64_t E,
                        int32_t* counts, int32_t* offsets, int32_t* perm, void* stream);

/* Workspace bytes tsa_moe_prefill needs. */
int tsa_moe_prefill_workspace_size(const tsa_expert_layout* layout, int64_t T, int k, int64_t E,
                                   int64_t* bytes);

/* Batched prefill: tokens grouped by expert, one grouped dequant-GEMM per phase on MFMA,
 * then the weighted combine out[t] = sum_j weights[t, j] * y_(t,j). Tiled MXFP4 pools (bf16
 * x) run fp4 x fp6 (or bf16) GEMMs; GGUF pools (bf16 x, hidden and inter multiples of 256,
 * T k >= 64, block-aligned slots) run bf16 GEMMs on blocks decoded on the fly, as the
 * reference's batched GGUF expert casts its weights to bf16 (tinyserve/ggml_forward.py:
 * 117-151); other calls run the decode kernels over the assignments.
 * expert_slot [E] int32 maps expert id -> slot (-1: not resident, contributes zero);
 * idx [T, k] int32 expert ids. Replaces ExpertPipeline.execute_layer_experts_batched /
 * _execute_layer_experts_batched_native (tinyserve/expert_pipeline.py:166-239,287-337) and
 * ExpertBatcher.batch_execute (tinyserve/expert_batcher.py:31-85). */
int tsa_moe_prefill(const tsa_expert_layout* layout, const void* pool, int64_t n_slots,
                    const int32_t* expert_slot, int64_t E,
                    const int32_t* idx, const float* weights, int64_t T, int k,
                    const void* x, int x_dtype, void* y, int y_dtype,
                    void* workspace, int64_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TINYSERVE_AMD_H */
