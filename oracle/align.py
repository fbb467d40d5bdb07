"""moe_align_block_size (numpy).

Reference: the upstream vLLM op (schema
vllm_musa/patches/series/0041-MUSA-MUSA-csrc-csrc-moe-torch_bindings.cpp.patch:36-58,
C++ signature 0048-MUSA-MUSA-csrc-csrc-moe-moe_align_sum_kernels.cu.patch:49-56,
sizing max_num_tokens_padded = numel + E * (block - 1) as in
model_executor/layers/fused_moe/fused_moe.py:881-884): per-expert counts are
padded to a multiple of the block size, segments are laid out in expert order,
padding slots hold the sentinel numel, expert_ids[b] names the expert of
block b, num_tokens_post_pad is the padded total.  With an expert map, ids
map to local ids and routes of non-local experts are dropped.

The upstream kernel places routes with atomics, so the order inside a segment
is not defined there; this restatement fixes it to ascending route index (a
stable sort), and the GPU kernel follows the same rule.  Blocks past the used
range get expert id -1.
"""
from __future__ import annotations

import numpy as np


def capacity_for(numel: int, num_experts: int, block_size: int) -> int:
    return numel + num_experts * (block_size - 1)


def moe_align_block_size(topk_ids: np.ndarray, num_experts: int, block_size: int,
                         expert_map: np.ndarray | None = None, capacity: int | None = None):
    """Returns (sorted_token_ids, expert_ids, num_tokens_post_pad, expert_offsets, scatter_idx)."""
    ids = np.asarray(topk_ids).reshape(-1).astype(np.int64)
    numel = ids.size
    if capacity is None:
        capacity = capacity_for(numel, num_experts, block_size)
    e = ids.copy()
    if expert_map is not None:
        em = np.asarray(expert_map).astype(np.int64)
        ok = (e >= 0) & (e < em.size)
        e = np.where(ok, em[np.clip(e, 0, em.size - 1)], -1)
    e = np.where((e >= 0) & (e < num_experts), e, -1)
    valid = e >= 0
    counts = np.bincount(e[valid], minlength=num_experts)
    padded = (counts + block_size - 1) // block_size * block_size
    offsets = np.zeros(num_experts + 1, dtype=np.int64)
    offsets[1:] = np.cumsum(padded)
    total = int(offsets[-1])
    sorted_ids = np.full(capacity, numel, dtype=np.int32)
    scatter = np.full(numel, -1, dtype=np.int32)
    order = np.argsort(np.where(valid, e, num_experts), kind="stable")[: int(valid.sum())]
    # rank of each placed route inside its expert segment
    pe = e[order]
    starts = np.zeros(num_experts + 1, dtype=np.int64)
    starts[1:] = np.cumsum(counts)
    rank = np.arange(order.size) - starts[pe]
    pos = offsets[pe] + rank
    sorted_ids[pos] = order.astype(np.int32)
    scatter[order] = pos.astype(np.int32)
    nblocks = -(-capacity // block_size)
    expert_ids = np.full(nblocks, -1, dtype=np.int32)
    for ex in range(num_experts):
        b0, b1 = offsets[ex] // block_size, offsets[ex + 1] // block_size
        expert_ids[b0:b1] = ex
    return (sorted_ids, expert_ids, np.array([total], dtype=np.int32),
            offsets.astype(np.int32), scatter)
