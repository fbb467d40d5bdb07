/*
 * vllm_musa_amd.h -- C ABI of the MI355X (gfx950) quantized-MoE / block-fp8
 * matmul library (libvllm_musa_amd.so).
 *
 * Conventions (shared by every entry point):
 *   - Pointers are device pointers (hipMalloc'd or torch CUDA tensors);
 *     sizes are element counts; row-major, innermost stride 1 unless a
 *     stride argument says otherwise.
 *   - Work is enqueued on `stream` (a hipStream_t); nothing synchronises
 *     the host and no entry point allocates device memory.  Scratch memory,
 *     where needed, is passed in and sized by the matching *_workspace_size().
 *   - Each call returns VMAMD_OK (0) or an error code; the message of the
 *     last failure on the calling thread is returned by vmamd_last_error().
 *   - fp8 means OCP float8 e4m3fn (one byte per value); bf16 and f16 are
 *     passed as their 16-bit patterns.
 *
 * Each declaration names the reference interface (MooreThreads/vllm-musa,
 * file:line) that it replaces.
 */
#ifndef VLLM_MUSA_AMD_H_
#define VLLM_MUSA_AMD_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* vmamd_stream_t; /* == hipStream_t */

#define VMAMD_OK 0
#define VMAMD_ERR_INVALID 1 /* bad argument: shape, dtype, alignment, size */
#define VMAMD_ERR_HIP 2     /* a HIP runtime call or kernel launch failed   */

#define VMAMD_DTYPE_F32 0
#define VMAMD_DTYPE_F16 1
#define VMAMD_DTYPE_BF16 2
#define VMAMD_DTYPE_E8M0 3 /* unsigned power-of-two exponent byte (scales only) */
#define VMAMD_DTYPE_E4M3 4 /* OCP float8 e4m3fn operand (the GEMV ops)            */

/* Message of the last error on this thread ("" if none). */
const char* vmamd_last_error(void);
/* ABI version of the library (bumped on incompatible changes). */
int vmamd_abi_version(void);

/* ------------------------------------------------------------ quantizers --
 * Per-token-group fp8 quantisation of activations:
 *   s[r,g] = max(eps, max_{c in g} |x[r,c]|) / fp8_max
 *   q[r,c] = e4m3fn(clamp(x[r,c] / s[r,g], fp8_min, fp8_max))
 * x: [rows, cols] (bf16/f16/f32, row stride x_row_stride elements), q: [rows,
 * cols] contiguous fp8, s: scale of (row r, group g) at
 * s[r*s_stride_row + g*s_stride_group] (row-major: (cols/group, 1);
 * column-major: (1, rows)).  group_size must be 128.
 * Replaces per_token_group_quant_8bit_vec
 * (csrc/musa/quantization/per_token_group_quant_8bit_vec.cu:111-178) and the
 * Python per_token_group_quant_fp8
 * (vllm_musa/model_executor/layers/quantization/utils/fp8_utils.py:33-152).
 */
int vmamd_per_token_group_quant_fp8(const void* x, int x_dtype, int64_t rows, int64_t cols,
                                    int64_t x_row_stride, int group_size, float eps,
                                    float fp8_min, float fp8_max, void* q, float* s,
                                    int64_t s_stride_row, int64_t s_stride_group,
                                    vmamd_stream_t stream);

/* out[r, c] = silu(x[r, c]) * x[r, d + c] rounded to the activation dtype;
 * x: [rows, 2d], out: [rows, d].  Replaces torch.ops._C.silu_and_mul /
 * maybe_fast_silu_and_mul (vllm_musa/jit_kernel/csrc/moe.py:102-116). */
int vmamd_silu_and_mul(const void* x, int dtype, int64_t rows, int64_t d, void* out,
                       vmamd_stream_t stream);

/* SiLU-and-mul fused with the 1x128 fp8 group quantiser.  The product is
 * rounded to the activation dtype before quantisation.  swiglu_limit > 0
 * clamps gate <= L and up to [-L, L] (L rounded to the activation dtype).
 * x: [rows, 2d]; q: [rows, d] fp8; s: [rows, d/128] f32 row-major.
 * Replaces silu_and_mul_per_token_group_fp8_quant and
 * silu_and_mul_clamp_per_token_group_fp8_quant
 * (csrc/musa/quantization/silu_and_mul_per_token_group_fp8_quant.cu:133-213). */
int vmamd_silu_and_mul_quant_fp8(const void* x, int dtype, int64_t rows, int64_t d,
                                 int group_size, float eps, float fp8_min, float fp8_max,
                                 float swiglu_limit, void* q, float* s, vmamd_stream_t stream);

/* Per-row (per-token) fp8 quantisation: s[r] = max(eps, max_c |x[r,c]|) /
 * fp8_max over the whole row, q[r,c] = e4m3fn(clamp(x[r,c] / s[r], fp8_min,
 * fp8_max)).  x: [rows, cols] bf16 (row stride x_row_stride elements, 16-byte
 * aligned rows), q: [rows, cols] fp8 contiguous, s: [rows] f32.  cols must be
 * a multiple of 8 and at most 16384.  Replaces the dynamic per-row activation
 * quantisation of the w4afp8 MoE (vllm_musa/kernels/w4afp8_moe.py:47-78
 * _scatter_quantized_rows and 81-124 _swiglu_quantized_rows, eps 1e-4). */
int vmamd_per_token_quant_fp8(const void* x, int64_t rows, int64_t cols, int64_t x_row_stride,
                              float eps, float fp8_min, float fp8_max, void* q, float* s,
                              vmamd_stream_t stream);

/* ---------------------------------------------------------------- routing --
 * Softmax top-k.  l' = gating (+ bias[e] if bias != NULL), optionally
 * soft-capped (softcap > 0: l' = tanh(l'/softcap)*softcap).  ids = the top-k
 * of l' in descending order, ties to the lower expert id; weights =
 * softmax(l')[ids], renormalised over the selection when renormalize != 0.
 * gating: [tokens, experts] f32/f16/bf16; weights f32 and ids i32 [tokens, topk].
 * experts <= 1024.  token_expert_indices (NULL: not written): i32 [tokens,
 * topk] with [t, k] = k * tokens + t, the third output of upstream fused_topk
 * that its topk_softmax op writes in the same kernel.  Replaces topk_softmax
 * (vllm_musa/jit_kernel/csrc/topk.py:211-242; kernels
 * jit_kernel/csrc/topk/topk_gating.mu:63-147, 458-529, 612-702). */
int vmamd_topk_softmax(const void* gating, int dtype, int64_t tokens, int experts, int topk,
                       int renormalize, float softcap, const float* bias, float* topk_weights,
                       int32_t* topk_ids, int32_t* token_expert_indices, vmamd_stream_t stream);

/* Sigmoid top-k.  s = sigmoid(gating); ids = top-k of s (+ bias), ties to the
 * lower id; weights = s[ids], renormalised when renormalize != 0;
 * token_expert_indices as vmamd_topk_softmax.  Replaces topk_sigmoid
 * (vllm_musa/jit_kernel/csrc/topk.py:245-275). */
int vmamd_topk_sigmoid(const void* gating, int dtype, int64_t tokens, int experts, int topk,
                       int renormalize, const float* bias, float* topk_weights,
                       int32_t* topk_ids, int32_t* token_expert_indices, vmamd_stream_t stream);

/* Folded shared expert: out = [topk_weights | w_s], [topk_ids | shared_expert_id]
 * ([tokens, topk + 1]) with w_s = sigmoid(shared_logits[t]) computed in fp32
 * and rounded to the logit dtype (VMAMD_DTYPE_*).  The routed weights are
 * copied unchanged (no renormalisation with the shared weight).  Replaces
 * extend_topk_with_shared (vllm_musa/jit_kernel/extend_topk_shared.py:17-73)
 * and the shared column of the fused-shared top-k
 * (vllm_musa/jit_kernel/csrc/topk/topk_gating.mu:369-456). */
int vmamd_extend_topk_with_shared(const float* topk_weights, const int32_t* topk_ids,
                                  int64_t tokens, int topk, const void* shared_logits, int dtype,
                                  int32_t shared_expert_id, float* out_weights, int32_t* out_ids,
                                  vmamd_stream_t stream);

#define VMAMD_SCORING_SOFTMAX 0
#define VMAMD_SCORING_SIGMOID 1

/* Softmax / sigmoid top-k with the fused shared expert: as vmamd_topk_softmax
 * / vmamd_topk_sigmoid for the topk routed columns, plus column topk of each
 * [tokens, topk + 1] output row = the shared expert (weight = sigmoid of
 * shared_logits[t] in fp32, rounded to shared_dtype; id = shared_expert_id;
 * outside the renormalisation), written by the same kernel.  topk <= 63.
 * Replaces the shared1 variants of topk_softmax / topk_sigmoid
 * (vllm_musa/jit_kernel/csrc/topk/topk_gating.mu:369-456, jit_kernel/csrc/topk.py:35-100). */
int vmamd_topk_softmax_shared(const void* gating, int dtype, int64_t tokens, int experts, int topk,
                              int renormalize, float softcap, const float* bias,
                              const void* shared_logits, int shared_dtype,
                              int32_t shared_expert_id, float* topk_weights, int32_t* topk_ids,
                              vmamd_stream_t stream);
int vmamd_topk_sigmoid_shared(const void* gating, int dtype, int64_t tokens, int experts, int topk,
                              int renormalize, const float* bias, const void* shared_logits,
                              int shared_dtype, int32_t shared_expert_id, float* topk_weights,
                              int32_t* topk_ids, vmamd_stream_t stream);

/* Grouped top-k (DeepSeek-V3 routing).  scores = softmax or sigmoid of the
 * gating row; sel = scores + bias (bias may be NULL); group score = sum of
 * the top-2 sel in the group when bias != NULL, else the group max; keep the
 * topk_group best groups (ties to the lower group); ids = top-k of sel over
 * the kept groups (ties to the lower id); weights = scores[ids], renormalised
 * when renormalize != 0, times routed_scaling_factor.  experts <= 1024,
 * experts % num_expert_group == 0, experts / num_expert_group <= 64.
 * Replaces grouped_topk / _grouped_topk_general
 * (vllm_musa/model_executor/layers/fused_moe/router/grouped_topk_router.py:257-357,
 * 388-469) and the MATE moe_fused_gate call it makes (277-303). */
int vmamd_grouped_topk(const void* gating, int dtype, int64_t tokens, int experts,
                       int num_expert_group, int topk_group, int topk, int renormalize,
                       int scoring, float routed_scaling_factor, const float* bias,
                       float* topk_weights, int32_t* topk_ids, vmamd_stream_t stream);

/* ------------------------------------------------------------ align/sort --
 * moe_align_block_size.  Routes r = 0..numel-1 (r = token*topk + slot) are
 * grouped by expert (after expert_map, if given: entries < 0 drop the route;
 * ids >= num_experts are dropped too); each expert's segment is padded to a
 * multiple of block_size.  Within a segment routes keep ascending r.
 *   sorted_token_ids[0..capacity): route ids, padding = numel;
 *   expert_ids[b]: expert of block b, -1 past the used blocks
 *                  (array length ceil(capacity / block_size));
 *   num_tokens_post_pad[0] = sum_e ceil(cnt_e / block_size) * block_size;
 *   expert_offsets (optional, length num_experts + 1): segment starts;
 *   scatter_idx (optional, length numel): position of route r in
 *                sorted_token_ids, -1 for dropped routes;
 *   active_experts (optional, length num_experts) and num_active (optional,
 *                length 1, given together): the experts that received at
 *                least one route, ascending, and their count.
 * capacity must be >= numel + num_experts * (block_size - 1).
 * num_experts <= 1024.  Replaces moe_align_block_size
 * (schema: vllm_musa/patches/series/0041-MUSA-MUSA-csrc-csrc-moe-torch_bindings.cpp.patch:36-58;
 * signature: 0048-MUSA-MUSA-csrc-csrc-moe-moe_align_sum_kernels.cu.patch:49-56). */
int vmamd_moe_align_block_size(const int32_t* topk_ids, int64_t numel, int num_experts,
                               int block_size, const int32_t* expert_map,
                               int64_t expert_map_len, int32_t* sorted_token_ids,
                               int64_t capacity, int32_t* expert_ids,
                               int32_t* num_tokens_post_pad, int32_t* expert_offsets,
                               int32_t* scatter_idx, int32_t* active_experts,
                               int32_t* num_active, vmamd_stream_t stream);

/* moe_align_block_size (the outputs above, without scatter_idx) and the 1x128
 * fp8 quantiser of the layer's bf16 activations x [rows, cols] into xq
 * [rows, cols] e4m3 and row-major xs [rows, cols/128] f32 (eps 1e-10, fp8
 * range +-448; the bytes vmamd_per_token_group_quant_fp8 writes), as one
 * launch: the first two steps of the fp8 layer (vmamd_fused_moe_fp8 runs
 * them so), for callers that drive the stage entry points.  cols % 128 == 0,
 * xq 8-byte aligned.  Replaces the fused routing + 1x128 quantisation that
 * opens the reference's DeepGEMM prefill, deep_gemm_contig_preprocess_fp8_tilelang
 * (vllm_musa/jit_kernel/tilelang/deep_gemm_contig_preprocess.py:1105-1130,
 * called at model_executor/layers/fused_moe/fused_moe.py:898-910), which
 * also permutes x into route order; the grouped GEMMs here gather x rows by
 * route instead. */
int vmamd_moe_align_block_size_quant_fp8(const int32_t* topk_ids, int64_t numel, int num_experts,
                                         int block_size, const int32_t* expert_map,
                                         int64_t expert_map_len, int32_t* sorted_token_ids,
                                         int64_t capacity, int32_t* expert_ids,
                                         int32_t* num_tokens_post_pad, int32_t* expert_offsets,
                                         int32_t* active_experts, int32_t* num_active, const void* x,
                                         int64_t rows, int64_t cols, void* xq, float* xs,
                                         vmamd_stream_t stream);

/* ---------------------------------------------------------------- combine --
 * out[t, h] = round(sum_{k<topk} x[t, k, h]) with an fp32 accumulator in slot
 * order.  x: [tokens, topk, hidden], out: [tokens, hidden], same dtype.
 * topk_ids (optional, [tokens, topk] i32): slots with a negative id, or an id
 * that expert_map (optional, length expert_map_len) maps to a negative local
 * id, are skipped.
 * Replaces moe_sum (0041-…torch_bindings.cpp.patch:44-50) and
 * maybe_fast_moe_sum (vllm_musa/jit_kernel/csrc/moe.py:119-133;
 * jit_kernel/csrc/moe/moe_sum_reduce.mu:104-147). */
int vmamd_moe_sum(const void* x, int dtype, int64_t tokens, int topk, int64_t hidden,
                  const int32_t* topk_ids, const int32_t* expert_map, int64_t expert_map_len,
                  void* out, vmamd_stream_t stream);

/* Weighted top-k combine: out[t, h] = round(sum_k x[t, k, h] * w[t, k]), fp32
 * accumulator in slot order, one rounding; skipping rules as vmamd_moe_sum.
 * Replaces _combine_expert_rows (vllm_musa/kernels/w4afp8_moe.py:127-161) and
 * post_reorder_triton_kernel (vllm_musa/jit_kernel/post_reorder.py:13-44),
 * with an fp32 accumulator for both. */
int vmamd_moe_weighted_sum(const void* x, int dtype, int64_t tokens, int topk, int64_t hidden,
                           const float* topk_weights, const int32_t* topk_ids,
                           const int32_t* expert_map, int64_t expert_map_len, void* out,
                           vmamd_stream_t stream);

/* ------------------------------------------------------- block-fp8 GEMM --
 * C[M, N] = bf16( sum_kb (sum_{k in kb} A[m,k] B[n,k]) * As[m,kb] * Bs[n/128, kb] )
 * A [M, K] fp8 with As[m*as_stride_m + kb*as_stride_k] (1x128 groups),
 * B [N, K] fp8 with Bs [ceil(N/128), K/128] f32 (128x128 blocks), C [M, N]
 * bf16.  K % 128 == 0, N % 16 == 0, block_n == block_k == 128.  Small M
 * runs the split-K GEMV (weights read once, K split over the waves of a
 * workgroup and reduced in LDS), larger M the tiled MFMA GEMM; where its
 * tiles are too few to fill the GPU the GEMM splits K over workgroups into
 * fp32 partials held in `workspace` and adds them in split order (a second
 * kernel).  vmamd_w8a8_block_fp8_matmul_workspace_size() gives the bytes the
 * shape's plan needs (0 when it needs none; 16-byte aligned).  With a smaller
 * or NULL workspace the call still succeeds: M <= 64 then takes the GEMV
 * and larger M the unsplit GEMM, whose fp32 sums run in another order.
 * Results are deterministic for a given shape and workspace.  Replaces
 * w8a8_triton_block_scaled_mm(A, B, As, Bs, block_size, output_dtype) as
 * called at vllm_musa/deepseek_v4_jit/fp8_einsum.py:399-406 and fp8_gemm_nt in
 * _musa_deepgemm_fp8_op (model_executor/kernels/linear/scaled_mm/deep_gemm.py:233-262),
 * both W8A8: the activations arrive quantised.  The reference's small-M
 * musa_fused_gemv, which reads bf16 activations unquantised, is
 * vmamd_fused_gemv below. */
size_t vmamd_w8a8_block_fp8_matmul_workspace_size(int64_t M, int64_t N, int64_t K);
int vmamd_w8a8_block_fp8_matmul(const void* A, const float* As, int64_t as_stride_m,
                                int64_t as_stride_k, const void* B, const float* Bs, void* C,
                                int64_t M, int64_t N, int64_t K, int block_n, int block_k,
                                void* workspace, size_t workspace_bytes, vmamd_stream_t stream);

/* vmamd_w8a8_block_fp8_matmul for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * allocation).  It has no counterpart in the reference.  The same plan and
 * kernels, with the split-K partials in a fixed device-resident scratch array
 * of VMAMD_W8A8_NOALLOC_SCRATCH_BYTES per GPU (held by each GPU the library
 * runs on until the process ends) instead of a workspace; the call allocates
 * nothing.  A shape whose plan needs more partial bytes than that
 * (vmamd_w8a8_block_fp8_matmul_workspace_size) is rejected with
 * VMAMD_ERR_INVALID.  Results equal vmamd_w8a8_block_fp8_matmul's with a
 * sufficient workspace, bit for bit.  All calls on one GPU share its array:
 * calls that overlap on one GPU (different streams, or host threads) race. */
#define VMAMD_W8A8_NOALLOC_SCRATCH_BYTES (64ull << 20)
int vmamd_w8a8_block_fp8_matmul_noalloc(const void* A, const float* As, int64_t as_stride_m,
                                        int64_t as_stride_k, const void* B, const float* Bs,
                                        void* C, int64_t M, int64_t N, int64_t K, int block_n,
                                        int block_k, vmamd_stream_t stream);

/* ------------------------------------------------------------ fused MoE --
 * One fused-experts layer with 128x128 block-fp8 weights, the whole pipeline
 * on `stream`: 1x128 quantisation of x, moe_align_block_size, W13 grouped
 * GEMM, SiLU-and-mul (+ optional clamp) and 1x128 quantisation of the
 * intermediate, W2 grouped GEMM with the routed weight applied in its
 * epilogue, and the top-k combine:
 *   out[t] = bf16( sum_k bf16( W2[e] . q(bf16(silu(h_g) * h_u)) * w[t,k] ) ),
 *   h = bf16(W13[e] . q(x[t])),  e = (expert_map ? expert_map[id] : id)
 * x [T, H] bf16; w13 [E, 2I, H] fp8 (rows [0, I) gate, [I, 2I) up) with
 * w13_s [E, 2I/128, H/128] f32; w2 [E, H, I] fp8 with w2_s [E, H/128, I/128];
 * topk_weights f32 / topk_ids i32 [T, topk] (negative ids, ids mapped to a
 * negative local id, and local ids >= num_experts contribute nothing); out
 * [T, H] bf16.  swiglu_limit > 0 selects the clamped activation.
 * apply_router_weight_on_input != 0 moves the routed weight to the W13 output
 * (h = bf16((W13[e] . q(x[t])) * w[t,k]), y unweighted), as upstream
 * fused_experts_impl does with MUL_ROUTED_WEIGHT on its first GEMM.  path: AUTO picks the
 * decode (expert-major GEMV, weights streamed once) kernels while T*topk <=
 * 2.5*E (12*E for the bf16 and w4afp8 layers) and the prefill (grouped MFMA
 * GEMM) kernels above; GEMV / GEMM force one.  On the decode kernels one
 * token (top-k <= 16) skips the alignment: each route is its own GEMV slot,
 * x is quantised inside the W13 launch and the W2 launch sums the top-k
 * (same bits as the aligned form).  NATIVE_GEMV computes the layer with the
 * numerics of the reference's native GEMV-MoE instead (decode kernels only):
 * x is not quantised (bf16 x dequantised fp8), gate and up stay fp32 through
 * the SwiGLU (clamped with the limit rounded to bf16), and the routed weight
 * multiplies gate and up before it (apply_router_weight_on_input) or the W2
 * sum after it:
 *   out[t] = bf16( sum_k bf16( (W2[e] . a) * w[t,k] ) ),
 *   a = bf16(silu(g) * u), (g, u) = fp32 W13[e] . x[t]
 * Workspace: vmamd_fused_moe_fp8_workspace_size() bytes (for the same path),
 * 256-byte aligned.
 * Replaces fused_experts_impl / _musa_fused_experts_impl_dispatch
 * (vllm_musa/model_executor/layers/fused_moe/fused_moe.py:1935-2184,
 * 2214-2760) for use_fp8_w8a8 with block_shape [128, 128]: the W8A8
 * upstream Triton and DeepGEMM prefill (824-951) paths (AUTO / GEMV / GEMM),
 * and the driver loop over the native GEMV-MoE musa_fused_gemv_moe
 * (fused_moe.py:2126-2184, csrc/musa/gemv.mu:249-514) as NATIVE_GEMV. */
#define VMAMD_MOE_PATH_AUTO 0
#define VMAMD_MOE_PATH_GEMV 1
#define VMAMD_MOE_PATH_GEMM 2
#define VMAMD_MOE_PATH_NATIVE_GEMV 3
size_t vmamd_fused_moe_fp8_workspace_size(int64_t T, int topk, int num_experts, int64_t H,
                                          int64_t I, int path);
int vmamd_fused_moe_fp8(const void* x, int x_dtype, int64_t T, int64_t H, const void* w13,
                        const float* w13_s, const void* w2, const float* w2_s, int num_experts,
                        int64_t I, const float* topk_weights, const int32_t* topk_ids, int topk,
                        const int32_t* expert_map, int64_t expert_map_len, float swiglu_limit,
                        int apply_router_weight_on_input, int path, void* out, void* workspace,
                        size_t workspace_bytes, vmamd_stream_t stream);

/* ------------------------------------------------ fused-MoE fp8 stages --
 * The two grouped expert GEMMs of vmamd_fused_moe_fp8, callable one by one
 * over the outputs of vmamd_per_token_group_quant_fp8 (xq, xs) and
 * vmamd_moe_align_block_size (sorted_token_ids of length `capacity`,
 * expert_offsets, num_tokens_post_pad, and for block_m 16 active_experts /
 * num_active).  block_m selects the kernels and must equal the align call's
 * block_size: 16 = decode (expert-major GEMV, each weight row streamed once
 * per call), 128 = prefill (grouped MFMA GEMM over 128-route blocks), 256 =
 * long prefill (256-route blocks; same results as 128).  The fused call
 * takes 256 from 128 routes per expert (fp8 and bf16; bf16 also 320, see
 * below).
 *
 * W13:  a = bf16(silu(h_gate) * h_up), h = bf16(W13[e] . q(x[t])), then a is
 *       quantised per 1x128 group into a2q (fp8) / a2s (f32, [rows, I/128]).
 *       Rows of a2q/a2s are routes (r = t*topk + k, [T*topk, I]) for
 *       block_m 16, positions of sorted_token_ids ([capacity, I]) for 128 / 256.
 * W2:   y[r] = bf16(W2[e] . dequant(a2q[row(r)]) * topk_weights[r]),
 *       y [T*topk, H] bf16 (8-byte aligned; 16-byte for block_m 256 and 320); rows of
 *       dropped routes are left unwritten.
 * Scratch: vmamd_moe_fp8_stage_workspace_size() bytes, 16-byte aligned
 * (enough for either stage).  At block_m 256 (H / 128 a multiple of 4) it
 * holds W13's copy of the x scales in route order, capacity x H/128 floats;
 * given less, W13 reads the scales by token row instead (same result).
 * Replace the two invoke_fused_moe_kernel launches of the upstream
 * fused_experts_impl (block-scaled accumulate:
 * vllm_musa/patches/series/0081-MUSA-vllm.model_executor.layers.fused_moe.fused_moe.patch:64-108;
 * activation then a2 quantisation: 0144-…:62-78) and the two
 * m_grouped_fp8_gemm_nt_contiguous calls of the DeepGEMM prefill path
 * (vllm_musa/model_executor/layers/fused_moe/fused_moe.py:914-934). */
size_t vmamd_moe_fp8_stage_workspace_size(int64_t T, int topk, int num_experts, int64_t H,
                                          int64_t I, int block_m);
int vmamd_moe_fp8_w13(const void* xq, const float* xs, int64_t T, int64_t H, int topk,
                      const int32_t* sorted_token_ids, int64_t capacity, int block_m,
                      const int32_t* expert_offsets, const int32_t* num_tokens_post_pad,
                      const int32_t* active_experts, const int32_t* num_active, const void* w13,
                      const float* w13_s, int num_experts, int64_t I, float swiglu_limit,
                      void* a2q, float* a2s, void* workspace, size_t workspace_bytes,
                      vmamd_stream_t stream);
int vmamd_moe_fp8_w2(const void* a2q, const float* a2s, int64_t T, int topk,
                     const int32_t* sorted_token_ids, int64_t capacity, int block_m,
                     const int32_t* expert_offsets, const int32_t* num_tokens_post_pad,
                     const int32_t* active_experts, const int32_t* num_active, const void* w2,
                     const float* w2_s, int num_experts, int64_t H, int64_t I,
                     const float* topk_weights, const int32_t* topk_ids,
                     const int32_t* expert_map, int64_t expert_map_len, void* y,
                     void* workspace, size_t workspace_bytes, vmamd_stream_t stream);

/* ------------------------------------------------------------ bf16 MoE --
 * The same layer and stages with bf16 expert weights (the reference's
 * unquantised path: MusaUnquantizedFusedMoEMethod.forward_oot ->
 * fused_experts, vllm_musa/model_executor/layers/fused_moe/unquantized_fused_moe_method.py:81-130,
 * upstream Triton fused_moe_kernel in bf16):
 *   out[t] = bf16( sum_k bf16( W2[e] . a * w[t,k] ) ),
 *   a = bf16(silu(h_g) * h_u),  h = bf16(W13[e] . x[t])   (fp32 accumulation)
 * x [T, H] bf16; w13 [E, 2I, H] bf16; w2 [E, H, I] bf16; a2 bf16 rows as for
 * fp8 ([T*topk, I] for block_m 16, [capacity, I] for the grouped GEMMs).
 * block_m: 16, 128, 256, or 320 (bf16 only: 320-route blocks on the same
 * 256-row tiles, which the fused call takes from 128 routes per expert
 * where the expected largest expert, mean + 3 sqrt(mean) routes, needs
 * fewer 320-route blocks than 256-route ones, each counted 1.25x; same
 * results).  Routing,
 * expert_map, swiglu_limit, path and workspace rules as for fp8;
 * NATIVE_GEMV keeps gate and up in fp32 through the SwiGLU, as the
 * reference's native bf16 GEMV-MoE does (csrc/musa/gemv.mu:430-434, 477-487):
 *   a = bf16(silu(g) * u), (g, u) = fp32 W13[e] . x[t]. */
size_t vmamd_fused_moe_bf16_workspace_size(int64_t T, int topk, int num_experts, int64_t H,
                                           int64_t I, int path);
int vmamd_fused_moe_bf16(const void* x, int64_t T, int64_t H, const void* w13, const void* w2,
                         int num_experts, int64_t I, const float* topk_weights,
                         const int32_t* topk_ids, int topk, const int32_t* expert_map,
                         int64_t expert_map_len, float swiglu_limit,
                         int apply_router_weight_on_input, int path, void* out, void* workspace,
                         size_t workspace_bytes, vmamd_stream_t stream);
size_t vmamd_moe_bf16_stage_workspace_size(int64_t T, int topk, int num_experts, int64_t H,
                                           int64_t I, int block_m);
int vmamd_moe_bf16_w13(const void* x, int64_t T, int64_t H, int topk,
                       const int32_t* sorted_token_ids, int64_t capacity, int block_m,
                       const int32_t* expert_offsets, const int32_t* num_tokens_post_pad,
                       const int32_t* active_experts, const int32_t* num_active, const void* w13,
                       int num_experts, int64_t I, float swiglu_limit, void* a2, void* workspace,
                       size_t workspace_bytes, vmamd_stream_t stream);
int vmamd_moe_bf16_w2(const void* a2, int64_t T, int topk, const int32_t* sorted_token_ids,
                      int64_t capacity, int block_m, const int32_t* expert_offsets,
                      const int32_t* num_tokens_post_pad, const int32_t* active_experts,
                      const int32_t* num_active, const void* w2, int num_experts, int64_t H,
                      int64_t I, const float* topk_weights, const int32_t* topk_ids,
                      const int32_t* expert_map, int64_t expert_map_len, void* y, void* workspace,
                      size_t workspace_bytes, vmamd_stream_t stream);

/* ---------------------------------------------------------- w4afp8 MoE --
 * One MoE layer with signed int4 expert weights (two per byte, element 2j in
 * the low nibble of byte j) and bf16 scales per (output row, 128-K group),
 * fp8 activations with one dynamic scale per row:
 *   xq = q_row(x)                          (s = max(1e-4, absmax(row)) / 448)
 *   h  = bf16(sum_kb (xq . W13_int4[e]^T)_kb * s13[e, n, kb] * s_x)
 *   a  = bf16(silu(min(h_g, L)) * clamp(h_u, -L, L))   (no clamp if L <= 0)
 *   y  = bf16(sum_kb (q_row(a) . W2_int4[e]^T)_kb * s2[e, n, kb] * s_a)
 *   out[t] = bf16(sum_k y[t, k] * w[t, k])  (fp32 accumulator)
 * x [T, H] bf16; w13 [E, 2I, H/2] int8 with w13_s [E, 2I, H/128] bf16; w2
 * [E, H, I/2] int8 with w2_s [E, H, I/128] bf16 (both scale arrays 4-byte
 * aligned); topk / expert_map / path / workspace rules as
 * vmamd_fused_moe_fp8.  H, I <= 16384.
 * Replaces w4afp8_moe (vllm_musa/kernels/w4afp8_moe.py:164-362) and the MATE
 * S4FP8 grouped GEMMs it calls (283-318), reached from
 * MusaW4AFp8MoEMethod.apply (model_executor/layers/quantization/w4afp8.py:147-170). */
size_t vmamd_w4afp8_moe_workspace_size(int64_t T, int topk, int num_experts, int64_t H,
                                       int64_t I, int path);
int vmamd_w4afp8_moe(const void* x, int64_t T, int64_t H, const void* w13, const void* w13_s,
                     const void* w2, const void* w2_s, int num_experts, int64_t I,
                     const float* topk_weights, const int32_t* topk_ids, int topk,
                     const int32_t* expert_map, int64_t expert_map_len, float swiglu_limit,
                     int path, void* out, void* workspace, size_t workspace_bytes,
                     vmamd_stream_t stream);

/* ------------------------------------------------- reference GEMV ops --
 * The reference's native GEMVs with their numerics: the activations are read
 * as they are (bf16 against fp8 weights dequantised per 128x128 block, no
 * activation quantisation), sums in fp32, one bf16 rounding of the output.
 *
 * vmamd_fused_gemv_moe: A [rows, K]; B [E, N, K]; route r = row*topk + k
 * (r < rows*topk) uses expert e = topk_ids[r] and writes row r of C:
 *   acc = sum_kb B_scale[e, n/128, kb] * sum_{k in kb} A[row, k] * B[e, n, k]
 *   acc *= topk_weights[r]                    (mul_routed_weight != 0)
 *   use_swiglu: C [rows*topk, N/2] = bf16(g * sigmoid(g) * u), g = acc[n],
 *               u = acc[N/2 + n], after g <= L, u in [-L, L] when
 *               swiglu_limit L > 0 (L is rounded to bf16 for bf16 A)
 *   otherwise   C [rows*topk, N] = bf16(acc)
 * A: bf16 (B e4m3 with B_scale [E, ceil(N/128), K/128] f32, or B bf16 with
 * no scales) or e4m3 with A_scale [rows, K/128] f32 (then B e4m3 and the
 * products carry A_scale[row, kb] too).  topk_ids / topk_weights: i32 / f32
 * with rows*topk entries.  A route whose id is outside [0, E) gets a zero
 * row.  K % 128 == 0 (bf16 B: K % 64), N % 16 == 0 (use_swiglu: N % 32);
 * A, B, C 16-byte aligned.  Up to 16 routes run one GEMV slot per route; more
 * are grouped per expert (weights streamed once per 16 routes).  Workspace:
 * vmamd_fused_gemv_moe_workspace_size() bytes, 256-byte aligned.
 * Replaces musa_fused_gemv_moe (csrc/musa/gemv.mu:927-1170, kernel 249-514;
 * schema csrc/musa/torch_bindings.cpp:11-15). */
size_t vmamd_fused_gemv_moe_workspace_size(int64_t rows, int topk, int num_experts, int64_t N,
                                           int64_t K, int a_dtype, int b_dtype);
int vmamd_fused_gemv_moe(const void* A, int a_dtype, const float* A_scale, int64_t rows, int64_t K,
                         const void* B, int b_dtype, const float* B_scale, int num_experts,
                         int64_t N, const float* topk_weights, const int32_t* topk_ids, int topk,
                         int mul_routed_weight, int use_swiglu, float swiglu_limit, void* C,
                         void* workspace, size_t workspace_bytes, vmamd_stream_t stream);

/* vmamd_fused_gemv: the dense GEMV, C [M, N or N/2] = the rows of A against
 * one weight matrix B [N, K] (B_scale [ceil(N/128), K/128] for e4m3 B), with
 * the vmamd_fused_gemv_moe rules for one expert, topk 1 and no routed weight.
 * Workspace: vmamd_fused_gemv_workspace_size() bytes, 256-byte aligned.
 * Replaces musa_fused_gemv (csrc/musa/gemv.mu:723-925; schema
 * csrc/musa/torch_bindings.cpp:17-21) as _musa_fp8_small_m_gemv_op calls it
 * (vllm_musa/model_executor/kernels/linear/scaled_mm/deep_gemm.py:512-536). */
size_t vmamd_fused_gemv_workspace_size(int64_t M, int64_t N, int64_t K, int a_dtype, int b_dtype);
int vmamd_fused_gemv(const void* A, int a_dtype, const float* A_scale, int64_t M, int64_t K,
                     const void* B, int b_dtype, const float* B_scale, int64_t N, int use_swiglu,
                     void* C, void* workspace, size_t workspace_bytes, vmamd_stream_t stream);

/* ------------------------------------------------------ checkpoint scales --
 * Converts n weight scales from src_dtype (E8M0, F32 or BF16) to dst_dtype
 * (F32 or BF16), element for element:
 *   e8m0 -> f32 : bits = b << 23 (b = 0 gives +0.0, b = 255 gives +inf)
 *   f32 -> bf16 : round to nearest even, NaN -> 0x7fc0
 * When invalid_count is not null, the number of destination values that are
 * not finite and positive is ADDED to *invalid_count (the caller clears it).
 * src and dst are either the same buffer (equal element sizes) or disjoint.
 * Replaces _upcast_e8m0_to_fp32 / deepgemm_post_process_fp8_weight_block
 * (vllm_musa/model_executor/layers/quantization/utils/fp8_utils.py:13-30)
 * and the cast + check of MusaW4AFp8MoEMethod.process_weights_after_loading
 * (model_executor/layers/quantization/w4afp8.py:126-135). */
int vmamd_convert_scales(const void* src, int src_dtype, int64_t n, void* dst, int dst_dtype,
                         int32_t* invalid_count, vmamd_stream_t stream);

/* ------------------------------------------------------ router-gate GEMM --
 * logits[M, E] = x[M, K] . w[E, K]^T in IEEE fp32, with one fixed summation
 * order per logit (independent of M and of the launch): lane l of 64 runs a
 * fused-multiply-add chain over k = 2l + 128i + j (i ascending, j = 0, 1),
 * starting from +0, and the 64 partials are added by an xor butterfly
 * (p_l += p_{l^s}, s = 32, 16, 8, 4, 2, 1).  x: bf16 or f32, rows contiguous
 * (stride K); w: f32 [E, K] contiguous; y: f32 [M, E] contiguous.
 * K % 128 == 0, E <= 65535.  M = 0 is a no-op.
 * Replaces router_gate_fp32 / _router_gate_fp32_kernel
 * (vllm_musa/model_executor/layers/fused_moe/router/musa_router_gemm.py:140-266). */
int vmamd_router_gate_fp32(const void* x, int x_dtype, int64_t M, int64_t K, const float* w,
                           int64_t E, float* y, vmamd_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* VLLM_MUSA_AMD_H_ */
