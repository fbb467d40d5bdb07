"""torch-facing wrappers of the C ABI with the reference's op signatures.

Outputs are caller-allocated and written in place, as the reference's
``Tensor!`` schemas (csrc/musa/torch_bindings.cpp:9-273, and the upstream
``_moe_C`` schemas restated in
vllm_musa/patches/series/0041-MUSA-MUSA-csrc-csrc-moe-torch_bindings.cpp.patch:20-58).
Every call launches on torch's current stream and never synchronises.
"""
from __future__ import annotations

import torch

from . import _lib
from ._lib import call, check_cuda, dtype_code, ptr, stream_of

FP8_DTYPE = torch.float8_e4m3fn
FP8_MAX = float(torch.finfo(FP8_DTYPE).max)  # 448
FP8_MIN = -FP8_MAX
E8M0_DTYPE = getattr(torch, "float8_e8m0fnu", None)

# Scale encodings of vmamd_convert_scales (VMAMD_DTYPE_*): raw uint8 bytes are
# taken as e8m0 exponents, like torch.float8_e8m0fnu.
_SCALE_SRC = {torch.float32: 0, torch.bfloat16: 2, torch.uint8: 3}
if E8M0_DTYPE is not None:
    _SCALE_SRC[E8M0_DTYPE] = 3
_SCALE_DST = {torch.float32: 0, torch.bfloat16: 2}


def _contig(t: torch.Tensor, name: str) -> None:
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


# ------------------------------------------------------------- quantisers --
def per_token_group_quant_8bit_vec(input: torch.Tensor, output_q: torch.Tensor,
                                   output_s: torch.Tensor, group_size: int, eps: float,
                                   min_8bit: float, max_8bit: float) -> None:
    """Reference: per_token_group_quant_8bit_vec
    (csrc/musa/quantization/per_token_group_quant_8bit_vec.cu:111-178).  Row- or
    column-major scales are taken from output_s's strides."""
    check_cuda(input, output_q, output_s)
    if input.dim() != 2 or output_s.dim() != 2:
        raise ValueError("per_token_group_quant_8bit_vec expects 2-D input and scales")
    if input.stride(-1) != 1:
        raise ValueError("input groups must be contiguous")
    _contig(output_q, "output_q")
    if output_q.dtype != FP8_DTYPE or output_s.dtype != torch.float32:
        raise ValueError("output_q must be float8_e4m3fn and output_s float32")
    rows, cols = input.shape
    if tuple(output_q.shape) != (rows, cols) or tuple(output_s.shape) != (rows, cols // group_size):
        raise ValueError("output shapes do not match the input")
    call("vmamd_per_token_group_quant_fp8", ptr(input), dtype_code(input.dtype), rows, cols,
         input.stride(0), group_size, eps, min_8bit, max_8bit, ptr(output_q), ptr(output_s),
         output_s.stride(0), output_s.stride(1), stream_of(input))


def silu_and_mul(out: torch.Tensor, x: torch.Tensor) -> None:
    """Reference: torch.ops._C.silu_and_mul(out, x) / maybe_fast_silu_and_mul
    (vllm_musa/jit_kernel/csrc/moe.py:102-116)."""
    check_cuda(out, x)
    _contig(x, "x")
    _contig(out, "out")
    d = x.shape[-1] // 2
    if out.shape[-1] != d or out.dtype != x.dtype or x.numel() != 2 * out.numel():
        raise ValueError("silu_and_mul: out must be x[..., :d]-shaped with x's dtype")
    call("vmamd_silu_and_mul", ptr(x), dtype_code(x.dtype), x.numel() // (2 * d) if d else 0, d,
         ptr(out), stream_of(x))


def _silu_quant(input, output_q, output_s, group_size, eps, fp8_min, fp8_max, limit):
    check_cuda(input, output_q, output_s)
    for t, n in ((input, "input"), (output_q, "output_q"), (output_s, "output_s")):
        _contig(t, n)
    if input.dim() != 2:
        raise ValueError("input must be 2-D [rows, 2*hidden]")
    rows, d2 = input.shape
    d = d2 // 2
    if tuple(output_q.shape) != (rows, d) or tuple(output_s.shape) != (rows, d // group_size):
        raise ValueError("output shapes do not match the input")
    call("vmamd_silu_and_mul_quant_fp8", ptr(input), dtype_code(input.dtype), rows, d, group_size,
         eps, fp8_min, fp8_max, limit, ptr(output_q), ptr(output_s), stream_of(input))


def silu_and_mul_per_token_group_fp8_quant(input: torch.Tensor, output_q: torch.Tensor,
                                           output_s: torch.Tensor, group_size: int, eps: float,
                                           fp8_min: float, fp8_max: float) -> None:
    """Reference: silu_and_mul_per_token_group_fp8_quant
    (csrc/musa/quantization/silu_and_mul_per_token_group_fp8_quant.cu:197-203)."""
    _silu_quant(input, output_q, output_s, group_size, eps, fp8_min, fp8_max, 0.0)


def silu_and_mul_clamp_per_token_group_fp8_quant(input: torch.Tensor, output_q: torch.Tensor,
                                                 output_s: torch.Tensor, group_size: int,
                                                 eps: float, fp8_min: float, fp8_max: float,
                                                 swiglu_limit: float) -> None:
    """Reference: silu_and_mul_clamp_per_token_group_fp8_quant (same file, 205-213)."""
    if not (swiglu_limit > 0 and swiglu_limit < float("inf")):
        raise ValueError("swiglu_limit must be finite and positive.")
    _silu_quant(input, output_q, output_s, group_size, eps, fp8_min, fp8_max, swiglu_limit)


# ---------------------------------------------------------------- routing --
def _check_routing_out(topk_weights, topk_ids, gating_output):
    check_cuda(topk_weights, topk_ids, gating_output)
    _contig(gating_output, "gating_output")
    _contig(topk_weights, "topk_weights")
    _contig(topk_ids, "topk_ids")
    if topk_weights.dtype != torch.float32 or topk_ids.dtype != torch.int32:
        raise ValueError("topk_weights must be float32 and topk_ids int32")
    if gating_output.dim() != 2 or topk_weights.shape != topk_ids.shape or \
            topk_weights.shape[0] != gating_output.shape[0]:
        raise ValueError("routing shapes do not match")


def extend_topk_with_shared(topk_weights: torch.Tensor, topk_ids: torch.Tensor,
                            shared_logits: torch.Tensor, shared_expert_id: int,
                            out_weights: torch.Tensor | None = None,
                            out_ids: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """[T, K] routing -> [T, K + 1]: the folded shared expert as one more
    always-selected slot, weight sigmoid(shared logit) rounded to the logit
    dtype, id shared_expert_id; routed weights unchanged.
    Reference: extend_topk_with_shared (vllm_musa/jit_kernel/extend_topk_shared.py:49-73)."""
    check_cuda(topk_weights, topk_ids, shared_logits, out_weights, out_ids)
    t, k = topk_weights.shape
    if topk_ids.shape != (t, k) or topk_weights.dtype != torch.float32 or topk_ids.dtype != torch.int32:
        raise ValueError("topk_weights must be float32 and topk_ids int32, both [T, K]")
    logits = shared_logits.reshape(-1)
    if logits.numel() != t:
        raise ValueError(f"shared_logits must hold one logit per token ({t}), got {logits.numel()}")
    logits = logits.contiguous()
    if out_weights is None:
        out_weights = torch.empty((t, k + 1), dtype=torch.float32, device=topk_weights.device)
    if out_ids is None:
        out_ids = torch.empty((t, k + 1), dtype=torch.int32, device=topk_ids.device)
    if tuple(out_weights.shape) != (t, k + 1) or tuple(out_ids.shape) != (t, k + 1):
        raise ValueError("outputs must be [T, K + 1]")
    _contig(out_weights, "out_weights")
    _contig(out_ids, "out_ids")
    call("vmamd_extend_topk_with_shared", ptr(topk_weights.contiguous()), ptr(topk_ids.contiguous()),
         t, k, ptr(logits), dtype_code(logits.dtype), int(shared_expert_id), ptr(out_weights),
         ptr(out_ids), stream_of(topk_weights))
    return out_weights, out_ids


def _shared_logits(shared_expert_gate_output, tokens):
    """The shared gate logits as a contiguous [T] vector of the gate's dtype."""
    check_cuda(shared_expert_gate_output)
    logits = shared_expert_gate_output.reshape(-1)
    if logits.numel() != tokens:
        raise ValueError(f"shared_expert_gate_output has {logits.numel()} logits for {tokens} tokens")
    return logits.contiguous()


def _shared_columns(topk_weights, shared_expert_gate_output, num_fused_shared_experts):
    """Number of routed columns when the top-k also appends the fused shared
    expert (the reference's shared1 kernels take exactly one)."""
    if shared_expert_gate_output is None or num_fused_shared_experts <= 0:
        return topk_weights.shape[1], False
    if num_fused_shared_experts != 1:
        raise NotImplementedError("only one fused shared expert is supported")
    return topk_weights.shape[1] - 1, True


def _check_tei(tei: torch.Tensor | None, topk_ids: torch.Tensor) -> None:
    if tei is not None and (tei.shape != topk_ids.shape or tei.dtype != torch.int32
                            or not tei.is_contiguous() or tei.device != topk_ids.device):
        raise ValueError("token_expert_indices must be a contiguous int32 tensor shaped like topk_ids")


def topk_softmax(topk_weights: torch.Tensor, topk_ids: torch.Tensor, gating_output: torch.Tensor,
                 renormalize: bool = False, moe_softcapping: float = 0.0,
                 correction_bias: torch.Tensor | None = None,
                 shared_expert_gate_output: torch.Tensor | None = None,
                 num_fused_shared_experts: int = 0,
                 token_expert_indices: torch.Tensor | None = None) -> None:
    """Reference: topk_softmax (vllm_musa/jit_kernel/csrc/topk.py:211-242).  With a
    shared gate output and one fused shared expert, the last of the
    topk_weights.shape[1] columns is that expert (id = number of routed experts,
    weight = sigmoid of its gate, outside the renormalisation), as the fused-shared
    kernel writes it (csrc/topk/topk_gating.mu:369-456).  token_expert_indices
    (routed columns only) receives [t, k] = k * T + t from the same kernel, as
    upstream fused_topk's op fills it."""
    _check_routing_out(topk_weights, topk_ids, gating_output)
    if correction_bias is not None:
        check_cuda(correction_bias)
        if correction_bias.dtype != torch.float32 or correction_bias.numel() != gating_output.shape[1]:
            raise ValueError("correction_bias must be float32 [num_experts]")
    t, e = gating_output.shape
    k, shared = _shared_columns(topk_weights, shared_expert_gate_output, num_fused_shared_experts)
    if token_expert_indices is not None and shared:
        raise NotImplementedError("token_expert_indices with a fused shared expert")
    _check_tei(token_expert_indices, topk_ids)
    if shared:
        logits = _shared_logits(shared_expert_gate_output, t)
        call("vmamd_topk_softmax_shared", ptr(gating_output), dtype_code(gating_output.dtype), t,
             e, k, int(bool(renormalize)), float(moe_softcapping), ptr(correction_bias),
             ptr(logits), dtype_code(logits.dtype), e, ptr(topk_weights), ptr(topk_ids),
             stream_of(gating_output))
        return
    call("vmamd_topk_softmax", ptr(gating_output), dtype_code(gating_output.dtype), t, e,
         k, int(bool(renormalize)), float(moe_softcapping),
         ptr(correction_bias), ptr(topk_weights), ptr(topk_ids), ptr(token_expert_indices),
         stream_of(gating_output))


def topk_sigmoid(topk_weights: torch.Tensor, topk_ids: torch.Tensor, gating_output: torch.Tensor,
                 renormalize: bool = False, correction_bias: torch.Tensor | None = None,
                 shared_expert_gate_output: torch.Tensor | None = None,
                 num_fused_shared_experts: int = 0,
                 token_expert_indices: torch.Tensor | None = None) -> None:
    """Reference: topk_sigmoid (vllm_musa/jit_kernel/csrc/topk.py:245-275); the fused
    shared expert and token_expert_indices as for topk_softmax."""
    _check_routing_out(topk_weights, topk_ids, gating_output)
    if correction_bias is not None:
        check_cuda(correction_bias)
        if correction_bias.dtype != torch.float32 or correction_bias.numel() != gating_output.shape[1]:
            raise ValueError("correction_bias must be float32 [num_experts]")
    t, e = gating_output.shape
    k, shared = _shared_columns(topk_weights, shared_expert_gate_output, num_fused_shared_experts)
    if token_expert_indices is not None and shared:
        raise NotImplementedError("token_expert_indices with a fused shared expert")
    _check_tei(token_expert_indices, topk_ids)
    if shared:
        logits = _shared_logits(shared_expert_gate_output, t)
        call("vmamd_topk_sigmoid_shared", ptr(gating_output), dtype_code(gating_output.dtype), t,
             e, k, int(bool(renormalize)), ptr(correction_bias), ptr(logits),
             dtype_code(logits.dtype), e, ptr(topk_weights), ptr(topk_ids),
             stream_of(gating_output))
        return
    call("vmamd_topk_sigmoid", ptr(gating_output), dtype_code(gating_output.dtype), t, e, k,
         int(bool(renormalize)), ptr(correction_bias), ptr(topk_weights), ptr(topk_ids),
         ptr(token_expert_indices), stream_of(gating_output))


def grouped_topk_into(topk_weights: torch.Tensor, topk_ids: torch.Tensor,
                      gating_output: torch.Tensor, num_expert_group: int, topk_group: int,
                      renormalize: bool, scoring_func: str, routed_scaling_factor: float,
                      e_score_correction_bias: torch.Tensor | None) -> None:
    _check_routing_out(topk_weights, topk_ids, gating_output)
    bias = e_score_correction_bias
    if bias is not None:
        check_cuda(bias)
        if bias.dtype != torch.float32:
            bias = bias.float()
        bias = bias.contiguous()
    scoring = {"softmax": 0, "sigmoid": 1}.get(scoring_func)
    if scoring is None:
        raise ValueError(f"Unsupported scoring function: {scoring_func}")
    t, e = gating_output.shape
    call("vmamd_grouped_topk", ptr(gating_output), dtype_code(gating_output.dtype), t, e,
         num_expert_group, topk_group, topk_weights.shape[1], int(bool(renormalize)), scoring,
         float(routed_scaling_factor), ptr(bias), ptr(topk_weights), ptr(topk_ids),
         stream_of(gating_output))


# ------------------------------------------------------------ align / sum --
def moe_align_block_size(topk_ids: torch.Tensor, num_experts: int, block_size: int,
                         sorted_token_ids: torch.Tensor, experts_ids: torch.Tensor,
                         num_tokens_post_pad: torch.Tensor,
                         maybe_expert_map: torch.Tensor | None = None,
                         scatter_idx: torch.Tensor | None = None,
                         expert_offsets: torch.Tensor | None = None,
                         active_experts: torch.Tensor | None = None,
                         num_active: torch.Tensor | None = None) -> None:
    """Reference: _moe_C.moe_align_block_size (schema
    patches/series/0041-…torch_bindings.cpp.patch:36-58).  Optional extra
    outputs: ``expert_offsets`` ([num_experts + 1] int32 segment starts) and
    ``active_experts`` / ``num_active`` (the experts with routes, ascending)."""
    check_cuda(topk_ids, sorted_token_ids, experts_ids, num_tokens_post_pad, maybe_expert_map,
               scatter_idx, expert_offsets, active_experts, num_active)
    if topk_ids.dtype != torch.int32:
        raise ValueError("topk_ids must be int32")
    for t, n in ((topk_ids, "topk_ids"), (sorted_token_ids, "sorted_token_ids"),
                 (experts_ids, "experts_ids")):
        _contig(t, n)
    cap = sorted_token_ids.numel()
    if experts_ids.numel() < -(-cap // block_size):
        raise ValueError("experts_ids is shorter than ceil(len(sorted_token_ids) / block_size)")
    emap = None if maybe_expert_map is None else maybe_expert_map.to(torch.int32).contiguous()
    call("vmamd_moe_align_block_size", ptr(topk_ids), topk_ids.numel(), num_experts, block_size,
         ptr(emap), 0 if emap is None else emap.numel(), ptr(sorted_token_ids), cap,
         ptr(experts_ids), ptr(num_tokens_post_pad), ptr(expert_offsets), ptr(scatter_idx),
         ptr(active_experts), ptr(num_active), stream_of(topk_ids))


def moe_align_block_size_quant_fp8(topk_ids: torch.Tensor, num_experts: int, block_size: int,
                                   sorted_token_ids: torch.Tensor, experts_ids: torch.Tensor,
                                   num_tokens_post_pad: torch.Tensor, x: torch.Tensor,
                                   output_q: torch.Tensor, output_s: torch.Tensor,
                                   maybe_expert_map: torch.Tensor | None = None,
                                   expert_offsets: torch.Tensor | None = None,
                                   active_experts: torch.Tensor | None = None,
                                   num_active: torch.Tensor | None = None) -> None:
    """moe_align_block_size and the 1x128 fp8 quantiser of bf16 x [rows, cols]
    (eps 1e-10, row-major scales) in one launch, with the outputs of the two
    separate ops: the opening of the fp8 layer, as the fused call runs it."""
    check_cuda(topk_ids, sorted_token_ids, experts_ids, num_tokens_post_pad, x, output_q, output_s,
               maybe_expert_map, expert_offsets, active_experts, num_active)
    if topk_ids.dtype != torch.int32:
        raise ValueError("topk_ids must be int32")
    for t, n in ((topk_ids, "topk_ids"), (sorted_token_ids, "sorted_token_ids"),
                 (experts_ids, "experts_ids"), (x, "x"), (output_q, "output_q"),
                 (output_s, "output_s")):
        _contig(t, n)
    if x.dim() != 2 or x.dtype != torch.bfloat16:
        raise ValueError("x must be a bf16 [rows, cols] tensor")
    rows, cols = x.shape
    if output_q.dtype != FP8_DTYPE or tuple(output_q.shape) != (rows, cols) or \
            output_s.dtype != torch.float32 or tuple(output_s.shape) != (rows, cols // 128):
        raise ValueError("output_q must be float8_e4m3fn [rows, cols] and output_s float32 "
                         "[rows, cols/128]")
    cap = sorted_token_ids.numel()
    if experts_ids.numel() < -(-cap // block_size):
        raise ValueError("experts_ids is shorter than ceil(len(sorted_token_ids) / block_size)")
    emap = None if maybe_expert_map is None else maybe_expert_map.to(torch.int32).contiguous()
    call("vmamd_moe_align_block_size_quant_fp8", ptr(topk_ids), topk_ids.numel(), num_experts,
         block_size, ptr(emap), 0 if emap is None else emap.numel(), ptr(sorted_token_ids), cap,
         ptr(experts_ids), ptr(num_tokens_post_pad), ptr(expert_offsets), ptr(active_experts),
         ptr(num_active), ptr(x), rows, cols, ptr(output_q), ptr(output_s), stream_of(x))


def moe_sum(input: torch.Tensor, output: torch.Tensor, topk_ids: torch.Tensor | None = None,
            expert_map: torch.Tensor | None = None) -> None:
    """Reference: _moe_C.moe_sum (schema 0041-…torch_bindings.cpp.patch:44-50) and
    maybe_fast_moe_sum (vllm_musa/jit_kernel/csrc/moe.py:119-133)."""
    check_cuda(input, output, topk_ids, expert_map)
    _contig(input, "input")
    _contig(output, "output")
    if input.dim() != 3 or output.dim() != 2 or input.shape[0] != output.shape[0] or \
            input.shape[2] != output.shape[1] or input.dtype != output.dtype:
        raise ValueError("moe_sum expects input [T, K, H] and output [T, H] of one dtype")
    ids = None if topk_ids is None else topk_ids.to(torch.int32).contiguous()
    emap = None if expert_map is None else expert_map.to(torch.int32).contiguous()
    t, k, h = input.shape
    call("vmamd_moe_sum", ptr(input), dtype_code(input.dtype), t, k, h, ptr(ids), ptr(emap),
         0 if emap is None else emap.numel(), ptr(output), stream_of(input))


def lib_version() -> int:
    return _lib.load().vmamd_abi_version()


def per_token_quant_fp8(x: torch.Tensor, eps: float = 1e-4) -> tuple[torch.Tensor, torch.Tensor]:
    """Dynamic per-row fp8 quantisation of bf16 x [rows, cols]: one scale
    max(eps, absmax(row)) / 448 per row (the w4afp8 activation quantiser,
    vllm_musa/kernels/w4afp8_moe.py:47-78).  Returns (q e4m3fn, s f32 [rows])."""
    check_cuda(x)
    if x.dim() != 2 or x.dtype != torch.bfloat16 or x.stride(-1) != 1:
        raise ValueError("per_token_quant_fp8 expects a bf16 [rows, cols] tensor with unit "
                         "column stride")
    rows, cols = x.shape
    q = torch.empty(rows, cols, dtype=FP8_DTYPE, device=x.device)
    s = torch.empty(rows, dtype=torch.float32, device=x.device)
    call("vmamd_per_token_quant_fp8", ptr(x), rows, cols, x.stride(0), eps, FP8_MIN, FP8_MAX,
         ptr(q), ptr(s), stream_of(x))
    return q, s


def moe_weighted_sum(input: torch.Tensor, topk_weights: torch.Tensor, output: torch.Tensor,
                     topk_ids: torch.Tensor | None = None,
                     expert_map: torch.Tensor | None = None) -> None:
    """output[t] = round(sum_k input[t, k] * topk_weights[t, k]) with an fp32
    accumulator in slot order (_combine_expert_rows, vllm_musa/kernels/w4afp8_moe.py:127-161)."""
    check_cuda(input, topk_weights, output, topk_ids, expert_map)
    _contig(input, "input")
    _contig(output, "output")
    if input.dim() != 3 or output.shape != (input.shape[0], input.shape[2]) or \
            input.dtype != output.dtype:
        raise ValueError("moe_weighted_sum expects input [T, K, H] and output [T, H] of one dtype")
    w = topk_weights.to(torch.float32).contiguous()
    if w.shape != input.shape[:2]:
        raise ValueError("topk_weights must be [T, K]")
    ids = None if topk_ids is None else topk_ids.to(torch.int32).contiguous()
    emap = None if expert_map is None else expert_map.to(torch.int32).contiguous()
    t, k, h = input.shape
    call("vmamd_moe_weighted_sum", ptr(input), dtype_code(input.dtype), t, k, h, ptr(w), ptr(ids),
         ptr(emap), 0 if emap is None else emap.numel(), ptr(output), stream_of(input))


# ------------------------------------------------------ checkpoint scales --
def convert_scales(src: torch.Tensor, dst: torch.Tensor,
                   invalid_count: torch.Tensor | None = None) -> None:
    """dst = src converted element for element (e8m0 / f32 / bf16 -> f32 / bf16;
    e8m0 byte b -> float bits b << 23, f32 -> bf16 round to nearest even).  When
    given, invalid_count (one int32) is increased by the number of dst values
    that are not finite and positive.  References: _upcast_e8m0_to_fp32
    (quantization/utils/fp8_utils.py:13-15) and the cast + check of
    MusaW4AFp8MoEMethod.process_weights_after_loading
    (quantization/w4afp8.py:126-131)."""
    check_cuda(src, dst, invalid_count)
    _contig(src, "src")
    _contig(dst, "dst")
    if src.dtype not in _SCALE_SRC:
        raise ValueError(f"convert_scales: unsupported source dtype {src.dtype}")
    if dst.dtype not in _SCALE_DST:
        raise ValueError(f"convert_scales: unsupported destination dtype {dst.dtype}")
    if src.numel() != dst.numel():
        raise ValueError(f"convert_scales: {src.numel()} source and {dst.numel()} destination "
                         "elements")
    if invalid_count is not None and (invalid_count.dtype != torch.int32
                                      or invalid_count.numel() != 1):
        raise ValueError("invalid_count must be a single int32")
    call("vmamd_convert_scales", ptr(src), _SCALE_SRC[src.dtype], src.numel(), ptr(dst),
         _SCALE_DST[dst.dtype], ptr(invalid_count), stream_of(dst))


# ------------------------------------------------------- router-gate GEMM --
def router_gate_fp32(x: torch.Tensor, weight: torch.Tensor, out: torch.Tensor) -> None:
    """out[M, E] = x[M, K] . weight[E, K]^T in fp32 with a fixed, batch-invariant
    summation order (x bf16 or f32, weight f32, K % 128 == 0).  Reference:
    _router_gate_fp32_kernel (fused_moe/router/musa_router_gemm.py:140-226)."""
    check_cuda(x, weight, out)
    if x.dim() != 2 or weight.dim() != 2 or out.dim() != 2:
        raise ValueError("router_gate_fp32 expects 2-D x, weight and out")
    for t, name in ((x, "x"), (weight, "weight"), (out, "out")):
        _contig(t, name)
    m, k = x.shape
    e = weight.shape[0]
    if weight.shape[1] != k or tuple(out.shape) != (m, e):
        raise ValueError(f"router_gate_fp32: x {tuple(x.shape)}, weight {tuple(weight.shape)}, "
                         f"out {tuple(out.shape)} do not match")
    if weight.dtype != torch.float32 or out.dtype != torch.float32:
        raise ValueError("router_gate_fp32: weight and out must be float32")
    if x.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("router_gate_fp32: x must be float32 or bfloat16")
    call("vmamd_router_gate_fp32", ptr(x), dtype_code(x.dtype), m, k, ptr(weight), e, ptr(out),
         stream_of(x))


# ------------------------------------------------------ reference GEMV ops --
# musa_fused_gemv_moe / musa_fused_gemv with the reference's argument order
# and numerics (csrc/musa/gemv.mu:249-514, 723-1170; Python wrappers
# vllm_musa/_custom_ops.py:28-158): the activations are read as they are --
# bf16 against the fp8 weights dequantised per 128x128 block, no activation
# quantisation -- the sums are fp32 and the output is rounded once to bf16.
# Checks the reference's native op makes with TORCH_CHECK raise RuntimeError,
# as there; the asserts of its Python wrapper stay asserts.  The GEMV's own
# tile request (block_n, block_k) is checked by the reference's rules
# (gemv.mu:1037-1066) and then left to this library, which sizes its
# launches itself: it is a performance hint there and changes no value.
def _gemv_operand_dtype(t: torch.Tensor) -> int:
    if t.dtype == torch.bfloat16:
        return _lib.DTYPE_BF16
    if t.dtype == FP8_DTYPE:
        return _lib.DTYPE_E4M3
    raise NotImplementedError(f"GEMV operands of dtype {t.dtype} are not on this path "
                              "(bf16 activations, fp8 or bf16 weights)")


def _check_requested_block(block_n: int, block_k: int, nr_n: int, hidden: int, vlen: int) -> None:
    if (block_n == 0) != (block_k == 0):
        raise RuntimeError("requested GEMV block must provide both block_n and block_k, got "
                           f"{block_n}x{block_k}")
    if block_n == 0:
        return
    if not (block_n > 0 and block_k > 0 and block_n * block_k <= 512):
        raise RuntimeError("requested GEMV block must use positive sizes with block_n * "
                           f"block_k <= 512, got {block_n}x{block_k}")
    if nr_n % block_n or hidden % (block_k * vlen):
        raise RuntimeError(f"requested GEMV block={block_n}x{block_k} is invalid for "
                           f"nr_n={nr_n}, hidden_size={hidden}, vlen={vlen}")


def _gemv_common(A, B, C, A_scale, B_scale, rows, K, N, use_swigelu):
    """Shared argument checks; returns (a_dtype, b_dtype, A_scale, B_scale)
    as the C ABI takes them."""
    check_cuda(A, B, C, A_scale, B_scale)
    for t, n in ((A, "A"), (B, "B"), (C, "C")):
        _contig(t, n)
    a_dt, b_dt = _gemv_operand_dtype(A), _gemv_operand_dtype(B)
    if C.dtype != torch.bfloat16:
        raise RuntimeError("the GEMV output C must be bfloat16")
    if b_dt == _lib.DTYPE_E4M3:
        if B_scale is None or B_scale.dtype != torch.float32:
            raise RuntimeError("fp8 weights need float32 block scales")
        B_scale = B_scale.contiguous()
    else:
        B_scale = None  # bf16 weights take no scales (gemv.mu:430-434)
    if a_dt == _lib.DTYPE_E4M3:
        if b_dt != _lib.DTYPE_E4M3:
            raise RuntimeError("fp8 activations take fp8 weights")
        if A_scale is None or A_scale.dtype != torch.float32 or \
                A_scale.numel() != rows * (K // 128):
            raise RuntimeError("fp8 activations need float32 1x128 group scales [rows, K/128]")
        A_scale = A_scale.contiguous()
    else:
        A_scale = None  # bf16 activations are read as they are (gemv.mu:405-419)
    n_out = N // 2 if use_swigelu else N
    return a_dt, b_dt, A_scale, B_scale, n_out


def musa_fused_gemv_moe(A: torch.Tensor, B: torch.Tensor, C: torch.Tensor,
                        A_scale: torch.Tensor | None, B_scale: torch.Tensor | None,
                        topk_weights: torch.Tensor, topk_ids: torch.Tensor,
                        mul_routed_weight: bool, topk: int, use_int4_w4a16: bool,
                        use_swigelu: bool, block_n: int = 0, block_k: int = 0,
                        swiglu_limit: float = 0.0) -> None:
    """Reference: musa_fused_gemv_moe (vllm_musa/_custom_ops.py:28-59; op
    csrc/musa/gemv.mu:927-1170).  A [rows, K]; B [E, N, K]; route
    r = row * topk + k uses expert topk_ids.flat[r] and writes row r of C
    ([rows * topk, N], or [rows * topk, N/2] with use_swigelu: gate rows
    [0, N/2), up rows [N/2, N), silu(g) * u in fp32 with the clamp
    swiglu_limit rounded to A's dtype).  mul_routed_weight multiplies the fp32
    sums by topk_weights.flat[r] first.  An id outside [0, E) gives a zero
    row.  The fused-MoE driver calls it twice per layer: W13 over the tokens
    (topk = K, SwiGLU) and W2 over cache2's rows (topk = 1)."""
    if use_int4_w4a16:
        raise NotImplementedError("the int4 W4A16 GEMV-MoE is not on this path")
    if A.dim() != 2:
        raise RuntimeError("A must be dim 2.")
    if B.dim() != 3:
        raise RuntimeError("B must be dim 3.")
    rows, K = A.shape
    E, N, Kb = B.shape
    if Kb != K:
        raise RuntimeError(f"A has K={K}, B has K={Kb}")
    vlen = 16 if B.dtype == FP8_DTYPE else 8
    _check_requested_block(int(block_n), int(block_k), N // 2 if use_swigelu else N, K, vlen)
    a_dt, b_dt, A_scale, B_scale, n_out = _gemv_common(A, B, C, A_scale, B_scale, rows, K, N,
                                                       use_swigelu)
    check_cuda(A, topk_weights, topk_ids)
    if topk_ids.dtype != torch.int32 or topk_ids.numel() != rows * topk:
        raise RuntimeError(f"topk_ids must be int32 with rows * topk = {rows * topk} entries")
    if topk_weights.dtype != torch.float32 or topk_weights.numel() != rows * topk:
        raise RuntimeError("topk_weights must be float32 with rows * topk entries")
    if C.numel() != rows * topk * n_out:
        raise RuntimeError(f"C must hold rows * topk x {n_out} elements")
    if B_scale is not None and tuple(B_scale.shape) != (E, -(-N // 128), K // 128):
        raise RuntimeError(f"B_scale must be [E, ceil(N/128), K/128] = {(E, -(-N // 128), K // 128)}")
    ids = topk_ids.contiguous()
    wts = topk_weights.contiguous()
    lib = _lib.load()
    nbytes = lib.vmamd_fused_gemv_moe_workspace_size(rows, topk, E, N, K, a_dt, b_dt)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=A.device)
    call("vmamd_fused_gemv_moe", ptr(A), a_dt, ptr(A_scale), rows, K, ptr(B), b_dt, ptr(B_scale), E,
         N, ptr(wts), ptr(ids), int(topk), int(bool(mul_routed_weight)), int(bool(use_swigelu)),
         float(swiglu_limit), ptr(C), ptr(ws), nbytes, stream_of(A))


def musa_fused_gemv_op(A: torch.Tensor, B: torch.Tensor, C: torch.Tensor,
                       A_scale: torch.Tensor | None, B_scale: torch.Tensor | None,
                       use_int4_w4a16: bool, use_swigelu: bool, use_rms_norm: bool,
                       gamma: torch.Tensor | None, eps: float) -> None:
    """The raw op musa_fused_gemv in its schema's argument order
    (csrc/musa/torch_bindings.cpp:17-21; gemv.mu:723-925): C [M, N or N/2] =
    A [M, K] against one weight matrix B [N, K] (B_scale [ceil(N/128),
    K/128] for fp8), as _musa_fp8_small_m_gemv_op calls it
    (scaled_mm/deep_gemm.py:512-536)."""
    if use_int4_w4a16:
        raise NotImplementedError("the int4 W4A16 GEMV is not on this path")
    if use_rms_norm:
        raise NotImplementedError("the GEMV's fused RMS norm is not on this path")
    if A.dim() != 2:
        raise RuntimeError("A must be dim 2.")
    if B.dim() != 2:
        raise RuntimeError("B must be dim 2.")
    M, K = A.shape
    N, Kb = B.shape
    if Kb != K:
        raise RuntimeError(f"A has K={K}, B has K={Kb}")
    a_dt, b_dt, A_scale, B_scale, n_out = _gemv_common(A, B, C, A_scale, B_scale, M, K, N,
                                                       use_swigelu)
    if tuple(C.shape) != (M, n_out):
        raise RuntimeError(f"C must be [M, {n_out}]")
    if B_scale is not None and tuple(B_scale.shape) != (-(-N // 128), K // 128):
        raise RuntimeError("B_scale must be [ceil(N/128), K/128]")
    lib = _lib.load()
    nbytes = lib.vmamd_fused_gemv_workspace_size(M, N, K, a_dt, b_dt)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=A.device)
    call("vmamd_fused_gemv", ptr(A), a_dt, ptr(A_scale), M, K, ptr(B), b_dt, ptr(B_scale), N,
         int(bool(use_swigelu)), ptr(C), ptr(ws), nbytes, stream_of(A))


def musa_fused_gemv(x: torch.Tensor, qweight: torch.Tensor, x_scales: torch.Tensor | None = None,
                    qweight_scales: torch.Tensor | None = None, use_swigelu: bool = False,
                    use_rms_norm: bool = False, gamma: torch.Tensor | None = None,
                    eps: float = 1e-6, output: torch.Tensor | None = None) -> torch.Tensor:
    """Reference: the Python wrapper musa_fused_gemv (vllm_musa/_custom_ops.py:62-158):
    fp8 weights with block scales write into ``output`` (allocated when None,
    else checked), bf16 weights into a new tensor of x's dtype."""
    out_shape = x.shape[:-1] + (qweight.shape[0] if not use_swigelu else qweight.shape[0] // 2,)
    assert not (use_swigelu and use_rms_norm), "gemv only fused one activation (swigelu or rms_norm)!"
    if use_rms_norm and gamma is None:
        raise AssertionError("rms_norm gamm is None!")
    if qweight.dtype == FP8_DTYPE:
        assert qweight_scales is not None, "FP8 grouped matmul weight scales is None!"
        if output is None:
            output = torch.empty(out_shape, device=x.device, dtype=torch.bfloat16)
        else:
            assert output.shape == out_shape
            assert output.device == x.device
            assert output.dtype == torch.bfloat16
            assert output.is_contiguous()
        musa_fused_gemv_op(x, qweight, output, x_scales, qweight_scales, False, use_swigelu,
                           use_rms_norm, gamma, eps)
        return output
    if qweight_scales is not None:
        raise NotImplementedError("the int4 W4A16 GEMV is not on this path")
    assert output is None, "caller-owned output is only supported for FP8 GEMV"
    output = torch.empty(out_shape, device=x.device, dtype=x.dtype)
    musa_fused_gemv_op(x, qweight, output, None, None, False, use_swigelu, use_rms_norm, gamma, eps)
    return output


# The same two ops as torch.ops._C_musa_ops.musa_fused_gemv_moe / musa_fused_gemv
# (schemas csrc/musa/torch_bindings.cpp:11-21), so call sites written against
# the reference's extension -- its fused-MoE driver and its dense small-M
# GEMV -- run unchanged; fake implementations let them be traced.
_OPS_NS = "_C_musa_ops"


def _register_reference_ops() -> None:
    ns = getattr(torch.ops, _OPS_NS)
    if not hasattr(ns, "musa_fused_gemv_moe"):
        moe = torch.library.custom_op(f"{_OPS_NS}::musa_fused_gemv_moe", mutates_args=("C",))(
            _gemv_moe_op_impl)
        moe.register_fake(_gemv_moe_op_fake)
    if not hasattr(ns, "musa_fused_gemv"):
        dense = torch.library.custom_op(f"{_OPS_NS}::musa_fused_gemv", mutates_args=("C",))(
            _gemv_op_impl)
        dense.register_fake(_gemv_op_fake)


def _gemv_moe_op_impl(A: torch.Tensor, B: torch.Tensor, C: torch.Tensor,
                      A_scale: torch.Tensor | None, B_scale: torch.Tensor | None,
                      topk_weights: torch.Tensor, topk_ids: torch.Tensor, mul_routed_weight: bool,
                      topk: int, use_int4_w4a16: bool, use_swigelu: bool, block_n: int = 0,
                      block_k: int = 0, swiglu_limit: float = 0.0) -> None:
    musa_fused_gemv_moe(A, B, C, A_scale, B_scale, topk_weights, topk_ids, mul_routed_weight,
                        topk, use_int4_w4a16, use_swigelu, block_n, block_k, swiglu_limit)


def _gemv_moe_op_fake(A, B, C, A_scale, B_scale, topk_weights, topk_ids, mul_routed_weight, topk,
                      use_int4_w4a16, use_swigelu, block_n=0, block_k=0, swiglu_limit=0.0) -> None:
    return None


def _gemv_op_impl(A: torch.Tensor, B: torch.Tensor, C: torch.Tensor, A_scale: torch.Tensor | None,
                  B_scale: torch.Tensor | None, use_int4_w4a16: bool, use_swigelu: bool,
                  use_rms_norm: bool, gamma: torch.Tensor | None, eps: float) -> None:
    musa_fused_gemv_op(A, B, C, A_scale, B_scale, use_int4_w4a16, use_swigelu, use_rms_norm, gamma,
                       eps)


def _gemv_op_fake(A, B, C, A_scale, B_scale, use_int4_w4a16, use_swigelu, use_rms_norm, gamma,
                  eps) -> None:
    return None


_register_reference_ops()
