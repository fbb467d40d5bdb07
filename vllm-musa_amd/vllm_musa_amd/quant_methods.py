"""The MoE quant-method ``apply`` hooks with the reference's signatures.

Each reads the expert weights from the layer object the way the reference
method does and runs this package's fused layer:

  Fp8MoEMethod.apply               vllm_musa/model_executor/layers/quantization/fp8.py:212-291
                                   (block fp8: w13_weight / w2_weight with
                                   w13_weight_scale_inv / w2_weight_scale_inv)
  UnquantizedFusedMoEMethod.forward_oot
                                   model_executor/layers/fused_moe/unquantized_fused_moe_method.py:81-130
  W4AFp8MoEMethod.apply            model_executor/layers/quantization/w4afp8.py:147-170
  W4AFp8MoEMethod loading          model_executor/layers/quantization/w4afp8.py:74-140

Shared experts that the caller delegates (shared_experts with an input) are
added to the routed output, as the reference does when the runner hands them
to the quant method.  Expert-parallel all-to-all managers are not part of this
single-GPU path; layer.expert_map selects the local experts.

Fp8MoEMethod also carries the block-grid padding of the intermediate
partition (maybe_roundup_sizes / create_weights, quantization/fp8.py:27-115):
the kernels take I in multiples of 128, and zero-filled padding rows / columns
contribute nothing to the layer output; and the shared-expert fold
(fold_shared_expert, quantization/fp8.py:118-185, 191-244): a shared MLP with
the routed experts' shapes and block format is appended as expert E, and apply
gives every token one more slot on it, weighted by sigmoid of the shared gate,
so routed and shared work run as one grouped GEMM chain.
"""
from __future__ import annotations

import math

import torch

from . import _custom_ops as ops
from .fused_moe import fused_experts_impl
from .w4afp8_moe import w4afp8_moe


def _add_shared(routed, shared_experts, shared_experts_input, x):
    if shared_experts is None:
        return routed
    inp = shared_experts_input if shared_experts_input is not None else x
    return routed + shared_experts(inp)


def _activation(layer) -> str:
    act = getattr(layer, "activation", "silu")
    return getattr(act, "value", act) if not isinstance(act, str) else act


def _round_up(value: int, multiple: int) -> int:
    return (value + multiple - 1) // multiple * multiple


class Fp8MoEMethod:
    """Block-fp8 (128x128 weight blocks, dynamic 1x128 activations) experts."""

    def __init__(self, block_shape=(128, 128), swiglu_limit: float | None = None,
                 block_quant: bool = True):
        self.block_shape = list(block_shape)
        self.swiglu_limit = swiglu_limit
        self.block_quant = block_quant

    def maybe_roundup_sizes(self, hidden_size: int, intermediate_size_per_partition: int,
                            act_dtype: torch.dtype, moe_parallel_config) -> tuple[int, int]:
        """Pads a tensor-parallel shard's intermediate size up to the block grid
        (lcm of the weight block sides), as the reference does for block-quantised
        experts with tp_size > 1 (quantization/fp8.py:27-72)."""
        if not (self.block_quant and getattr(moe_parallel_config, "tp_size", 1) > 1):
            return hidden_size, intermediate_size_per_partition
        block_n, block_k = (int(b) for b in self.block_shape)
        return hidden_size, _round_up(intermediate_size_per_partition, math.lcm(block_n, block_k))

    def create_weights(self, layer, num_experts: int, hidden_size: int,
                       intermediate_size_per_partition: int, params_dtype=None,
                       intermediate_size_unpadded: int | None = None, device="cuda"):
        """Allocates the expert stack on `layer`: w13_weight [E, 2I, H] and
        w2_weight [E, H, I] in e4m3fn, w13_weight_scale_inv / w2_weight_scale_inv
        on the block grid.  When the partition was padded
        (intermediate_size_unpadded < I) the weights are zero-filled, so the
        padding rows and columns contribute nothing (quantization/fp8.py:75-115);
        padding-only scale blocks hold 1.0."""
        e, h, i = num_experts, hidden_size, intermediate_size_per_partition
        bn, bk = (int(b) for b in self.block_shape)
        fp8 = torch.float8_e4m3fn
        padded = intermediate_size_unpadded is not None and intermediate_size_unpadded != i
        alloc = torch.zeros if padded else torch.empty
        layer.w13_weight = alloc(e, 2 * i, h, dtype=fp8, device=device)
        layer.w2_weight = alloc(e, h, i, dtype=fp8, device=device)
        layer.w13_weight_scale_inv = torch.ones(e, -(-2 * i // bn), -(-h // bk), dtype=torch.float32,
                                                device=device)
        layer.w2_weight_scale_inv = torch.ones(e, -(-h // bn), -(-i // bk), dtype=torch.float32,
                                               device=device)
        layer.intermediate_size_per_partition = i
        layer.intermediate_size_unpadded = intermediate_size_unpadded or i

    @staticmethod
    def load_expert(layer, expert: int, w13, w13_scale, w2, w2_scale):
        """Copies one expert's unpadded checkpoint tensors (w13 [2*I0, H] gate
        then up, w2 [H, I0], block scales on their own grid) into the padded
        stack: gate rows at [0, I0), up rows at [I, I + I0), w2 columns
        [0, I0).  I0 must be a multiple of the block side, as the checkpoint's
        blocks do not straddle the shard boundary then."""
        i = layer.intermediate_size_per_partition
        i0 = w2.shape[1]
        bn = -(-layer.w13_weight.shape[1] // layer.w13_weight_scale_inv.shape[1])
        bk = -(-layer.w2_weight.shape[2] // layer.w2_weight_scale_inv.shape[2])
        if i0 % bn or i0 % bk:
            raise ValueError(f"unpadded intermediate size {i0} is not on the {bn}x{bk} block grid")
        layer.w13_weight[expert, :i0] = w13[:i0]
        layer.w13_weight[expert, i:i + i0] = w13[i0:]
        layer.w2_weight[expert, :, :i0] = w2
        nb0 = i0 // bn
        layer.w13_weight_scale_inv[expert, :nb0] = w13_scale[:nb0]
        layer.w13_weight_scale_inv[expert, i // bn:i // bn + nb0] = w13_scale[nb0:]
        layer.w2_weight_scale_inv[expert, :, :i0 // bk] = w2_scale

    weight_scale_name = "weight_scale_inv"

    def fold_shared_expert(self, layer, mlp) -> None:
        """Append the shared MLP (mlp.gate_up_proj [2I, H] gate-then-up rows and
        mlp.down_proj [H, I], each with its weight_scale_inv block scales) to the
        routed stack as expert E, release the shared projections, and mark the
        layer folded (layer._musa_shared_expert_id = E).  The shared expert must
        have a routed expert's shapes, dtypes and scale grid; once per layer,
        after loading.  Reference: _fold_shared_expert_weights
        (quantization/fp8.py:118-185)."""
        if mlp is None or getattr(layer, "_musa_shared_folded", False):
            return
        if getattr(layer, "expert_map", None) is not None:
            raise RuntimeError("shared-expert fold: expert parallelism is not folded")
        name = self.weight_scale_name
        parts = (("w13_weight", f"w13_{name}", mlp.gate_up_proj),
                 ("w2_weight", f"w2_{name}", mlp.down_proj))
        folded = {}
        for weight_attr, scale_attr, proj in parts:
            routed_w, routed_s = getattr(layer, weight_attr), getattr(layer, scale_attr)
            shared_w, shared_s = proj.weight, getattr(proj, name)
            if tuple(shared_w.shape) != tuple(routed_w.shape[1:]) or shared_w.dtype != routed_w.dtype:
                raise RuntimeError(f"shared-expert fold: {weight_attr} expects "
                                   f"{tuple(routed_w.shape[1:])}/{routed_w.dtype}, shared expert has "
                                   f"{tuple(shared_w.shape)}/{shared_w.dtype}")
            if tuple(shared_s.shape) != tuple(routed_s.shape[1:]) or shared_s.dtype != routed_s.dtype:
                raise RuntimeError(f"shared-expert fold: {scale_attr} expects "
                                   f"{tuple(routed_s.shape[1:])}/{routed_s.dtype}, shared expert has "
                                   f"{tuple(shared_s.shape)}/{shared_s.dtype}")
            folded[weight_attr] = torch.cat([routed_w, shared_w.unsqueeze(0)], dim=0).contiguous()
            folded[scale_attr] = torch.cat([routed_s, shared_s.unsqueeze(0)], dim=0).contiguous()
        num_routed = int(layer.w13_weight.shape[0])
        for attr, t in folded.items():
            setattr(layer, attr, t)
        for _, _, proj in parts:  # the shared projections now live in the stack
            proj.weight = None
            setattr(proj, name, None)
        layer._musa_shared_expert_id = num_routed
        layer._musa_shared_folded = True

    def apply(self, layer, x: torch.Tensor, topk_weights: torch.Tensor, topk_ids: torch.Tensor,
              shared_experts=None, shared_experts_input: torch.Tensor | None = None):
        if getattr(layer, "_musa_shared_folded", False):
            # The folded shared expert is one more always-selected slot; a router
            # that already appended it (top-k + 1 columns) is taken as is
            # (reference: apply, quantization/fp8.py:222-244).
            if shared_experts is not None or shared_experts_input is not None:
                raise ValueError("a folded shared expert expects shared_experts=None")
            routed_topk = int(getattr(getattr(layer, "moe_config", None), "experts_per_token",
                                      topk_ids.shape[1]))
            if topk_ids.shape[1] == routed_topk:
                shared_logits, _ = layer._musa_shared_gate(x)
                topk_weights, topk_ids = ops.extend_topk_with_shared(
                    topk_weights, topk_ids, shared_logits.reshape(-1), layer._musa_shared_expert_id)
            elif topk_ids.shape[1] != routed_topk + 1 or topk_weights.shape[1] != routed_topk + 1:
                raise ValueError(f"routing has {topk_ids.shape[1]} columns; expected {routed_topk} "
                                 f"or {routed_topk + 1} with the shared slot")
        routed = fused_experts_impl(
            x, layer.w13_weight, layer.w2_weight, topk_weights, topk_ids,
            activation=_activation(layer),
            apply_router_weight_on_input=getattr(layer, "apply_router_weight_on_input", False),
            use_fp8_w8a8=True, expert_map=getattr(layer, "expert_map", None),
            w1_scale=layer.w13_weight_scale_inv, w2_scale=layer.w2_weight_scale_inv,
            block_shape=self.block_shape, gemm1_clamp_limit=self.swiglu_limit)
        return _add_shared(routed, shared_experts, shared_experts_input, x)


class UnquantizedFusedMoEMethod:
    """bf16 experts."""

    def __init__(self, swiglu_limit: float | None = None):
        self.swiglu_limit = swiglu_limit

    def forward_oot(self, layer, x: torch.Tensor, topk_weights: torch.Tensor,
                    topk_ids: torch.Tensor, shared_experts=None,
                    shared_experts_input: torch.Tensor | None = None):
        routed = fused_experts_impl(
            x, layer.w13_weight, layer.w2_weight, topk_weights, topk_ids,
            activation=_activation(layer),
            apply_router_weight_on_input=getattr(layer, "apply_router_weight_on_input", False),
            expert_map=getattr(layer, "expert_map", None), gemm1_clamp_limit=self.swiglu_limit)
        return _add_shared(routed, shared_experts, shared_experts_input, x)

    apply = forward_oot


class W4AFp8MoEMethod:
    """Packed int4 experts with bf16 group-128 scales and dynamic per-row fp8
    activations.

    Loading follows the reference method (quantization/w4afp8.py:74-140):
    create_weights allocates w13_weight [E, 2I, H/2] and w2_weight [E, H, I/2]
    int8 (two int4 per byte), float32 group-128 scales w13_weight_scale_inv
    [E, 2I, H/128] / w2_weight_scale_inv [E, H, I/128] and unused bf16
    input-scale placeholders; load_weight copies a tensor-parallel rank's shard
    of one checkpoint tensor; process_weights_after_loading casts the scales
    to bf16 on the GPU and rejects any that is not finite and positive."""

    GROUP = 128

    def __init__(self, swiglu_limit: float | None = None):
        self.swiglu_limit = swiglu_limit

    def maybe_roundup_sizes(self, hidden_size: int, intermediate_size_per_partition: int,
                            act_dtype: torch.dtype, moe_parallel_config) -> tuple[int, int]:
        """No padding: the int4 scale groups must not straddle a shard, so H and
        the partition's I must be multiples of 128 (quantization/w4afp8.py:74-87)."""
        if hidden_size % self.GROUP or intermediate_size_per_partition % self.GROUP:
            raise ValueError(
                f"W4AFP8 experts need H and I per partition in multiples of {self.GROUP} "
                f"(got H={hidden_size}, I={intermediate_size_per_partition}); a tensor-parallel "
                "split that breaks the groups needs --enable-expert-parallel instead")
        return hidden_size, intermediate_size_per_partition

    def create_weights(self, layer, num_experts: int, hidden_size: int,
                       intermediate_size_per_partition: int, params_dtype=None, device="cuda",
                       **extra_weight_attrs) -> None:
        """Registers the packed weights, float32 scales and input-scale
        placeholders on `layer` (quantization/w4afp8.py:89-124); extra
        attributes (weight_loader, ...) are set on every parameter and the scales
        carry quant_method = "group"."""
        e, h, i, g = num_experts, hidden_size, intermediate_size_per_partition, self.GROUP
        shapes = {"w13_weight": (e, 2 * i, h // 2), "w2_weight": (e, h, i // 2),
                  "w13_weight_scale_inv": (e, 2 * i, h // g), "w2_weight_scale_inv": (e, h, i // g),
                  "w13_input_scale": (e,), "w2_input_scale": (e,)}
        for name, shape in shapes.items():
            if name.endswith("weight"):
                value, attrs = torch.empty(shape, dtype=torch.int8, device=device), extra_weight_attrs
            else:
                fill = torch.ones if name.endswith("input_scale") else torch.empty
                dtype = torch.bfloat16 if name.endswith("input_scale") else torch.float32
                value = fill(shape, dtype=dtype, device=device)
                attrs = {**extra_weight_attrs, "quant_method": "group"}
            param = torch.nn.Parameter(value, requires_grad=False)
            for key, attr in attrs.items():
                setattr(param, key, attr)
            if isinstance(layer, torch.nn.Module):
                layer.register_parameter(name, param)
            else:
                setattr(layer, name, param)
        layer.intermediate_size_per_partition = i

    @staticmethod
    def load_weight(layer, name: str, loaded_weight: torch.Tensor, expert_id: int, shard_id: str,
                    tp_rank: int = 0, tp_size: int = 1) -> None:
        """Copies tensor-parallel rank tp_rank's shard of one expert's checkpoint
        tensor into `layer`.  w1 / w3 (gate / up: [I, H/2] packed weights, [I,
        H/128] scales) are split along dim 0 and land in the first / second half
        of the w13 rows; w2 ([H, I/2], [H, I/128]) is split along dim 1.  The
        input-scale placeholders are ignored: activations are quantised
        dynamically.  Same shards as vLLM's fused-MoE loader
        (_load_w13 / _load_w2, exercised by tests/test_w4afp8_quantization.py:228-293)."""
        if name.endswith("input_scale"):
            return
        if not 0 <= tp_rank < tp_size:
            raise ValueError(f"tp_rank {tp_rank} is outside tp_size {tp_size}")
        dest = getattr(layer, name).data[expert_id]
        if shard_id in ("w1", "w3"):
            if not name.startswith("w13"):
                raise ValueError(f"shard {shard_id} belongs to w13, not {name}")
            half = dest.shape[0] // 2
            if tuple(loaded_weight.shape) != (half * tp_size, dest.shape[1]):
                raise ValueError(f"{name}/{shard_id}: checkpoint shape {tuple(loaded_weight.shape)}, "
                                 f"expected {(half * tp_size, dest.shape[1])}")
            src = loaded_weight.narrow(0, half * tp_rank, half)
            dest = dest.narrow(0, half if shard_id == "w3" else 0, half)
        elif shard_id == "w2":
            if not name.startswith("w2"):
                raise ValueError(f"shard w2 belongs to w2, not {name}")
            cols = dest.shape[1]
            if tuple(loaded_weight.shape) != (dest.shape[0], cols * tp_size):
                raise ValueError(f"{name}/w2: checkpoint shape {tuple(loaded_weight.shape)}, "
                                 f"expected {(dest.shape[0], cols * tp_size)}")
            src = loaded_weight.narrow(1, cols * tp_rank, cols)
        else:
            raise ValueError(f"unknown shard id {shard_id!r}")
        dest.copy_(src)

    def process_weights_after_loading(self, layer) -> None:
        """Scales -> bf16 (round to nearest even) on the GPU; a scale that is not
        finite and positive after the cast raises ValueError naming its tensor
        (quantization/w4afp8.py:126-135)."""
        for name in ("w13_weight_scale_inv", "w2_weight_scale_inv"):
            src = getattr(layer, name).data.contiguous()
            dst = torch.empty(src.shape, dtype=torch.bfloat16, device=src.device)
            bad = torch.zeros(1, dtype=torch.int32, device=src.device)
            ops.convert_scales(src, dst, bad)
            if int(bad.item()):
                raise ValueError(f"Invalid W4AFP8 weight scale in {name}")
            setattr(layer, name, torch.nn.Parameter(dst, requires_grad=False))

    def apply(self, layer, x: torch.Tensor, topk_weights: torch.Tensor, topk_ids: torch.Tensor,
              shared_experts=None, shared_experts_input: torch.Tensor | None = None):
        if getattr(layer, "apply_router_weight_on_input", False):
            raise NotImplementedError("W4AFP8 router weights must apply to the output")
        routed = w4afp8_moe(x, layer.w13_weight, layer.w2_weight, layer.w13_weight_scale_inv,
                            layer.w2_weight_scale_inv, topk_weights, topk_ids,
                            getattr(layer, "expert_map", None), swiglu_limit=self.swiglu_limit)
        return _add_shared(routed, shared_experts, shared_experts_input, x)
