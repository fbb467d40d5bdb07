"""Benchmark of the fp8 block-quantised fused-MoE layer on one MI355X.

Workload (the headline line): one DeepSeek-V3-shape MoE layer -- E=256 routed
experts, grouped sigmoid+bias routing (8 groups, top-4 groups, top-8 experts,
renormalised, x2.5), H=7168, I=2048, W13/W2 in e4m3fn with 128x128 block
scales, activations quantised per 1x128 group -- at T=4096 tokens.  A step is
routing (grouped_topk) + fused_experts_impl over one batch whose inputs are
already in HBM.  Synthetic data: weights ~N(0, 0.02) quantised per block,
activations ~N(0, 1), logits ~N(0, 1), score bias ~N(0, 0.1).

Printed (rank 0, one JSON line): value = algorithmic TFLOP/s of the layer at
T=4096 (2*T*topk*3*H*I flops per call), ms_per_step from HIP events around the
K timed steps; `roofline` is the dominant kernel (W13 grouped GEMM at T=4096)
timed on its own with HIP events on its launch stream, its `traffic` (HBM
bytes per launch) and `mfma_util` read from the committed rocprofv3 counter
summaries; `cpu_baseline` times the torch CPU restatement of the layer on a
bounded sample of the same layer.  The other configurations of the metric are
extra keys, each point the median of --sweep-iters HIP-event timings after 10
warm-ups with cold weights (a 1 GiB buffer is read before each call), with
us / TFLOP/s / GB/s and the fraction of min(peak compute, AI x 8 TB/s):
  sweep      fp8 DeepSeek-V3 layer (this workload) at T = 1, 16, 256, 4096,
             also replayed from a HIP graph (`graph_us`, as a server runs decode)
  dense      w8a8 block-fp8 linear, (N, K) in (24576, 1536), (7168, 18432),
             (2112, 7168), (7168, 2048), M = 1, 4, 16, 64, 512, 4096: 1x128
             activation quantiser + GEMM (`us`) and the GEMM alone (`gemm_us`)
  bf16_moe   bf16 layer E=128, top-8 softmax renorm, H=2048, I=768 at
             T = 1, 16, 128, 1024, 8192, uniform and skewed (+2.0 on 8 experts)
  w4afp8_moe w4afp8 layer E=128, top-8, H=4096, I=1536 at T = 1, 32, 512, 4096
  native_gemv the reference's native GEMV-MoE numerics (bf16 activations
             against the fp8 weights) where its dispatcher runs them: fp8
             E=256, top-8, H=2048, I=128 at T = 1, 8, 13 (path auto), and the
             DeepSeek-V3 layer at T = 1 (path native_gemv); each beside the
             W8A8 decode kernels on the same call

  python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-sweep] [--no-cpu]
  python bench.py --traffic-probe   # the launches profiled for FETCH_SIZE / WRITE_SIZE
  python bench.py --dense           # dense block-fp8 linear shapes, M = 1 .. 4096 (JSON lines)
  python bench.py --w4              # w4afp8 MoE layer, T = 1, 32, 512, 4096 (JSON lines)
  python bench.py --swiglu          # clamped SwiGLU + block-fp8 down projection (JSON lines)
  python bench.py --fold            # shared expert folded into the MoE vs run as dense GEMMs
  python bench.py --native          # the native-GEMV numerics at their decode shapes (JSON lines)
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "vllm-musa_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

# MI355X published peaks (dense).
PEAK_HBM_GBS = 8000.0
PEAK_FP8_TFLOPS = 5000.0
PEAK_BF16_TFLOPS = 2500.0
WARMUP_SWEEP = 10

E, H, I, TOPK, GROUPS, TOPK_GROUP, SCALE = 256, 7168, 2048, 8, 8, 4, 2.5
T_HEADLINE = 4096
SWEEP_T = (1, 16, 256, 4096)
WEIGHT_SEED = 3000

METRIC = "fp8-block MoE layer µs, TFLOPS & HBM GB/s (% roofline) at T=1..4096"

# rocprofv3 counter summaries of the W13 kernel at T=4096: FETCH_SIZE and
# WRITE_SIZE per dispatch scaled by a 1 GiB copy ("traffic_bytes_per_launch:"
# fills roofline.traffic), and the fp8 MFMA counters ("mfma_util_w13:" fills
# roofline.mfma_util: MFMA flops per second over the dense fp8 peak).
TRAFFIC_SUMMARY = os.path.join("profiles", "gemm_traffic_large_t.md")
MFMA_SUMMARY = os.path.join("profiles", "mfma_utilisation_large_t.md")


def read_summary_value(rel: str, key: str, cast=int):
    path = os.path.join(ROOT, rel)
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith(key + ":"):
            return cast(line.split(":", 1)[1].strip())
    return None


def read_traffic() -> int | None:
    return read_summary_value(TRAFFIC_SUMMARY, "traffic_bytes_per_launch")


def layer_flops(routes: int) -> float:
    return 2.0 * routes * (2 * I * H + H * I)


def layer_bytes(t: int, used_experts: int) -> float:
    """Algorithmic HBM bytes of one layer call: each touched expert's fp8
    weights and block scales once, x (bf16) in, out (bf16) out, logits in,
    routing weights/ids out."""
    w = 3 * I * H + 4 * ((2 * I // 128) * (H // 128) + (H // 128) * (I // 128))
    return used_experts * w + 4.0 * t * H + 4.0 * t * E + 8.0 * t * TOPK


def w13_bytes(t: int, used_experts: int) -> float:
    """Algorithmic bytes of one W13 launch: touched experts' W13 + scales,
    fp8 x + scales in, fp8 a2 + scales out."""
    w = 2 * I * H + 4 * (2 * I // 128) * (H // 128)
    routes = t * TOPK
    return used_experts * w + t * (H + 4 * H // 128) + routes * (I + 4 * I // 128)


class Layer:
    def __init__(self, torch, t: int, weights):
        from vllm_musa_amd import synthetic
        self.torch = torch
        self.t = t
        self.w13, self.s13, self.w2, self.s2 = weights
        self.x = synthetic.activations(t, H, WEIGHT_SEED + 10 * t + 1)
        self.logits = synthetic.router_logits(t, E, WEIGHT_SEED + 10 * t + 2)
        self.bias = synthetic.score_bias(E, WEIGHT_SEED + 3)

    def route(self):
        from vllm_musa_amd import grouped_topk
        return grouped_topk(self.x, self.logits, TOPK, True, GROUPS, TOPK_GROUP, "sigmoid", SCALE,
                            self.bias)

    def step(self):
        from vllm_musa_amd.fused_moe import fused_experts_impl
        w, ids = self.route()
        return fused_experts_impl(self.x, self.w13, self.w2, w, ids, use_fp8_w8a8=True,
                                  w1_scale=self.s13, w2_scale=self.s2, block_shape=[128, 128])

    def used_experts(self) -> int:
        _, ids = self.route()
        return int(self.torch.unique(ids).numel())


def time_events(torch, fn, iters: int, flush=None) -> list[float]:
    """Per-call milliseconds from HIP events on the current stream; `flush`
    (untimed) runs before each call."""
    out = []
    for _ in range(iters):
        if flush is not None:
            flush()
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        fn()
        b.record()
        b.synchronize()
        out.append(a.elapsed_time(b))
    return out


def graph_median(torch, fn, iters: int, flush) -> float:
    """Median ms of one replay of `fn` captured in a HIP graph (how a serving
    engine runs decode steps: no host work between the kernels)."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn()
    for _ in range(3):
        graph.replay()
    torch.cuda.synchronize()
    ms = statistics.median(time_events(torch, graph.replay, iters, flush))
    del graph
    return ms


def cpu_baseline(torch, layer: Layer, max_experts: int = 16) -> dict:
    """The torch CPU restatement of the layer (oracle/moe_torch.py: float32
    contractions on dequantised operands, every host thread) on a bounded
    sample of the T=4096 layer: the routes of its most loaded experts, with
    their tokens and weights.  Median of 5 timed passes after 1 warm-up,
    reported in the layer's unit (TFLOP/s)."""
    import platform

    import numpy as np

    from oracle import moe_torch
    cores = os.cpu_count() or 1
    torch.set_num_threads(cores)
    w, ids = layer.route()
    ids_np = ids.cpu().numpy()
    counts = np.bincount(ids_np.ravel(), minlength=E)
    experts = np.argsort(-counts, kind="stable")[:max_experts]
    toks = np.nonzero(np.isin(ids_np, experts).any(axis=1))[0]
    # the sample's own expert stack: the chosen experts as 0..n-1, others dropped
    remap = np.full(E, -1, np.int64)
    remap[experts] = np.arange(experts.size)
    sub_ids = torch.from_numpy(remap[ids_np[toks]].astype(np.int64))
    sel = torch.from_numpy(experts.astype(np.int64)).to(layer.w13.device)
    u8 = lambda t: t.view(torch.uint8).index_select(0, sel).cpu()
    f32 = lambda t: t.index_select(0, sel).cpu()
    args = (layer.x.float().cpu()[torch.from_numpy(toks)], u8(layer.w13), f32(layer.s13),
            u8(layer.w2), f32(layer.s2), w.cpu()[torch.from_numpy(toks)], sub_ids)
    routes = int((sub_ids >= 0).sum())
    moe_torch.fused_experts_fp8(*args)
    times = []
    for _ in range(5):
        t0 = time.perf_counter()
        moe_torch.fused_experts_fp8(*args)
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    tflops = layer_flops(routes) / med / 1e12
    model = platform.processor() or "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(tflops, 6), "unit": "TFLOP/s", "cores": int(torch.get_num_threads()),
            "kind": "port", "cpu": model,
            "sample": f"torch float32 CPU restatement (oracle/moe_torch.py) of the T={layer.t} "
                      f"layer on its {experts.size} most loaded experts ({routes} routes of "
                      f"{toks.size} tokens), median of 5 after 1 warm-up = {med:.2f} s; the full "
                      f"layer extrapolates to {layer_flops(layer.t * TOPK) / (tflops * 1e12):.0f} s"}


# DeepSeek-V3 linear layers as [N, K] (fused q_a + kv_a, q_b, kv_b, o_proj,
# shared-expert gate_up and down, dense-FFN gate_up and down).
DENSE_SHAPES = ((2112, 7168), (24576, 1536), (32768, 512), (7168, 16384), (4096, 7168),
                (7168, 2048), (36864, 7168), (7168, 18432))
DENSE_M = (1, 4, 16, 32, 64, 128, 512, 4096)


def dense_sweep(torch, iters: int, log) -> int:
    """HIP-event medians of w8a8_block_fp8_matmul (caches flushed by a 1 GiB
    read before each call); bytes = weights + scales + activations + output."""
    from vllm_musa_amd import per_token_group_quant_fp8, synthetic
    from vllm_musa_amd.block_fp8 import w8a8_block_fp8_matmul
    flush_buf = torch.ones(1 << 28, dtype=torch.int32, device="cuda")
    for n, k in DENSE_SHAPES:
        w, ws = synthetic.dense_fp8_weight(n, k, 7)
        row = {"N": n, "K": k}
        for m in DENSE_M:
            x = synthetic.activations(m, k, 8)
            q, s = per_token_group_quant_fp8(x, 128)
            f = lambda: w8a8_block_fp8_matmul(q, w, s, ws, [128, 128])
            for _ in range(3):
                f()
            torch.cuda.synchronize()
            us = statistics.median(time_events(torch, f, iters, lambda: flush_buf.max())) * 1e3
            by = n * k + 4 * ((n + 127) // 128) * (k // 128) + m * k + 4 * m * (k // 128) + 2 * m * n
            fl = 2.0 * m * n * k
            row[f"M{m}"] = {"us": round(us, 1), "frac_hbm": round(by / (us * 1e-6) / (PEAK_HBM_GBS * 1e9), 3),
                            "frac_fp8_peak": round(fl / (us * 1e-6) / (PEAK_FP8_TFLOPS * 1e12), 3)}
        print(json.dumps(row), flush=True)
        del w, ws
    log("bench: dense sweep done")
    return 0


def fold_sweep(torch, weights, iters: int, log) -> int:
    """The headline layer plus one shared expert of the routed experts' shape:
    folded (Fp8MoEMethod.fold_shared_expert: expert E of the stack, one more
    slot per token weighted by sigmoid of the shared gate) vs the shared MLP as
    its own dense block-fp8 GEMMs (gate_up, SiLU-and-mul + quantiser, down) added
    to the routed output.  HIP-event medians, caches flushed before each call."""
    from types import SimpleNamespace

    from vllm_musa_amd import silu_mul_per_token_group_quant_fp8, synthetic
    from vllm_musa_amd.block_fp8 import apply_w8a8_block_fp8_linear, w8a8_block_fp8_matmul
    from vllm_musa_amd.fused_moe import fused_experts_impl
    from vllm_musa_amd.quant_methods import Fp8MoEMethod
    sw13, ss13, sw2, ss2 = synthetic.moe_fp8_weights(1, H, I, WEIGHT_SEED + 5)
    gate_vec = synthetic.activations(1, H, WEIGHT_SEED + 6).view(-1) * 0.02
    w13, s13, w2, s2 = weights
    layer = SimpleNamespace(w13_weight=w13, w2_weight=w2, w13_weight_scale_inv=s13,
                            w2_weight_scale_inv=s2, expert_map=None, activation="silu",
                            apply_router_weight_on_input=False,
                            moe_config=SimpleNamespace(experts_per_token=TOPK))
    layer._musa_shared_gate = lambda h: ((h @ gate_vec).view(-1, 1), None)
    mlp = SimpleNamespace(gate_up_proj=SimpleNamespace(weight=sw13[0].clone(), weight_scale_inv=ss13[0].clone()),
                          down_proj=SimpleNamespace(weight=sw2[0].clone(), weight_scale_inv=ss2[0].clone()))
    method = Fp8MoEMethod()
    method.fold_shared_expert(layer, mlp)
    flush_buf = torch.ones(1 << 28, dtype=torch.int32, device="cuda")
    for t in SWEEP_T:
        lay = Layer(torch, t, weights)

        def folded():
            w, ids = lay.route()
            return method.apply(layer, lay.x, w, ids)

        def separate():
            w, ids = lay.route()
            routed = fused_experts_impl(lay.x, w13, w2, w, ids, use_fp8_w8a8=True, w1_scale=s13,
                                        w2_scale=s2, block_shape=[128, 128])
            sig = torch.sigmoid(lay.x @ gate_vec).view(-1, 1)
            h = apply_w8a8_block_fp8_linear(lay.x, sw13[0], ss13[0])
            q, s = silu_mul_per_token_group_quant_fp8(h, 128)
            down = w8a8_block_fp8_matmul(q, sw2[0], s, ss2[0], [128, 128])
            return routed + down * sig

        row = {"T": t}
        for name, fn in (("folded_us", folded), ("separate_us", separate)):
            for _ in range(3):
                fn()
            torch.cuda.synchronize()
            row[name] = round(statistics.median(time_events(torch, fn, iters, lambda: flush_buf.max())) * 1e3, 1)
        row["speedup"] = round(row["separate_us"] / row["folded_us"], 3)
        print(json.dumps(row), flush=True)
        del lay
    log("bench: fold sweep done")
    return 0


# Down projections after a clamped SwiGLU, as [N, D] (gate_up is [M, 2D]):
# the dense MLP and the shared expert of a DeepSeek-V3-sized model.
SWIGLU_SHAPES = ((7168, 18432), (7168, 2048))
SWIGLU_M = (1, 16, 64, 4096)


def swiglu_sweep(torch, iters: int, log) -> int:
    """HIP-event medians of silu_clamp_block_fp8_matmul (quantiser + GEMM,
    caches flushed by a 1 GiB read before each call); algorithmic bytes = the
    bf16 gate_up read + weights and scales + the bf16 output."""
    from vllm_musa_amd import synthetic
    from vllm_musa_amd.block_fp8 import silu_clamp_block_fp8_matmul
    flush_buf = torch.ones(1 << 28, dtype=torch.int32, device="cuda")
    for n, d in SWIGLU_SHAPES:
        w, ws = synthetic.dense_fp8_weight(n, d, 7)
        row = {"N": n, "D": d}
        for m in SWIGLU_M:
            gate_up = synthetic.activations(m, 2 * d, 9)
            f = lambda: silu_clamp_block_fp8_matmul(gate_up, w, ws, 128, False, 10.0)
            for _ in range(3):
                f()
            torch.cuda.synchronize()
            us = statistics.median(time_events(torch, f, iters, lambda: flush_buf.max())) * 1e3
            by = 4 * m * d + n * d + 4 * ((n + 127) // 128) * (d // 128) + 2 * m * n
            fl = 2.0 * m * n * d
            row[f"M{m}"] = {"us": round(us, 1), "frac_hbm": round(by / (us * 1e-6) / (PEAK_HBM_GBS * 1e9), 3),
                            "frac_fp8_peak": round(fl / (us * 1e-6) / (PEAK_FP8_TFLOPS * 1e12), 3)}
        print(json.dumps(row), flush=True)
        del w, ws
    log("bench: swiglu sweep done")
    return 0


W4_E, W4_H, W4_I = 128, 4096, 1536


def w4_sweep(torch, iters: int, log) -> int:
    """The w4afp8 layer at T = 1, 32, 512, 4096 (w4_configs: routing +
    w4afp8_moe, HIP-event medians with caches flushed, graph replay), one JSON
    line per T."""
    flush_buf = torch.ones(1 << 28, dtype=torch.int32, device="cuda")
    for row in w4_configs(torch, iters, lambda: flush_buf.max(), log):
        print(json.dumps(row), flush=True)
    return 0


def point(us: float, flops: float, nbytes: float, peak_tflops: float) -> dict:
    """us / TFLOP/s / GB/s and the fractions of the roofline of one timed call."""
    ideal = max(flops / (peak_tflops * 1e12), nbytes / (PEAK_HBM_GBS * 1e9))
    return {"us": round(us, 1), "tflops": round(flops / (us * 1e-6) / 1e12, 2),
            "gbps": round(nbytes / (us * 1e-6) / 1e9, 1),
            "frac_hbm": round(nbytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4),
            "frac_peak": round(flops / (us * 1e-6) / 1e12 / peak_tflops, 4),
            "frac_roofline": round(ideal / (us * 1e-6), 4)}


def median_us(torch, fn, iters: int, flush) -> float:
    """Median HIP-event time (us) of `fn` after WARMUP_SWEEP warm-ups, caches
    flushed before each timed call."""
    for _ in range(WARMUP_SWEEP):
        fn()
    torch.cuda.synchronize()
    return statistics.median(time_events(torch, fn, iters, flush)) * 1e3


C1_SHAPES = ((24576, 1536), (7168, 18432), (2112, 7168), (7168, 2048))
C1_M = (1, 4, 16, 64, 512, 4096)


def dense_configs(torch, iters: int, flush, log) -> list:
    """Dense w8a8 block-fp8 linear at its benchmark shapes: the reference op
    (1x128 quantisation of bf16 A, then the block GEMM) and the GEMM alone.
    Bytes = N*K + 4*ceil(N/128)*(K/128) + 2*M*K + 2*M*N (A in bf16)."""
    from vllm_musa_amd import per_token_group_quant_fp8, synthetic
    from vllm_musa_amd.block_fp8 import apply_w8a8_block_fp8_linear, w8a8_block_fp8_matmul
    out = []
    for n, k in C1_SHAPES:
        w, ws = synthetic.dense_fp8_weight(n, k, 7)
        for m in C1_M:
            x = synthetic.activations(m, k, 8)
            q, s = per_token_group_quant_fp8(x, 128)
            wsz = n * k + 4 * ((n + 127) // 128) * (k // 128)
            fl = 2.0 * m * n * k
            us = median_us(torch, lambda: apply_w8a8_block_fp8_linear(x, w, ws), iters, flush)
            g_us = median_us(torch, lambda: w8a8_block_fp8_matmul(q, w, s, ws, [128, 128]), iters, flush)
            row = {"N": n, "K": k, "M": m, **point(us, fl, wsz + 2 * m * k + 2 * m * n, PEAK_FP8_TFLOPS)}
            g = point(g_us, fl, wsz + m * k + 4 * m * (k // 128) + 2 * m * n, PEAK_FP8_TFLOPS)
            row.update({"gemm_us": g["us"], "gemm_frac_roofline": g["frac_roofline"]})
            out.append(row)
        log(f"bench: dense {n}x{k} done")
        del w, ws
    return out


C2_E, C2_H, C2_I = 128, 2048, 768
C2_T = (1, 16, 128, 1024, 8192)


def bf16_configs(torch, iters: int, flush, log) -> list:
    """bf16 fused MoE (Qwen3-30B-A3B-like): routing (top-8 softmax renorm on
    ~N(0,1) logits, `skewed`: +2.0 on experts 0..7) + fused_experts_impl.
    Bytes = touched experts' W13 + W2 (bf16) + x in + out + logits + routing."""
    from vllm_musa_amd import fused_topk, synthetic
    from vllm_musa_amd.fused_moe import fused_experts_impl
    w13, w2 = synthetic.moe_bf16_weights(C2_E, C2_H, C2_I, 4000)
    out = []
    for skewed in (False, True):
        for t in C2_T:
            x = synthetic.activations(t, C2_H, 4001 + t)
            logits = synthetic.router_logits(t, C2_E, 4002 + t, hot=8 if skewed else 0)

            def step():
                w, ids, _ = fused_topk(x, logits, TOPK, True)
                return fused_experts_impl(x, w13, w2, w, ids)
            _, ids, _ = fused_topk(x, logits, TOPK, True)
            u = int(torch.unique(ids).numel())
            fl = 2.0 * t * TOPK * 3 * C2_H * C2_I
            by = u * 3 * C2_H * C2_I * 2 + 4.0 * t * C2_H + 4.0 * t * C2_E + 8.0 * t * TOPK
            row = {"T": t, "skewed": skewed, "experts_touched": u,
                   **point(median_us(torch, step, iters, flush), fl, by, PEAK_BF16_TFLOPS)}
            row["graph_us"] = round(graph_median(torch, step, iters, flush) * 1e3, 1)
            if t == C2_T[-1] and not skewed:
                row["kernels"] = bf16_kernels(torch, x, w13, w2, logits, iters, flush)
            out.append(row)
        log(f"bench: bf16 layer ({'skewed' if skewed else 'uniform'}) done")
    del w13, w2
    return out


def bf16_layer(torch, t: int, skewed: bool = False, weights=None):
    """The bf16 benchmark layer at T: (step, ids, weights); step = routing +
    fused_experts_impl."""
    from vllm_musa_amd import fused_topk, synthetic
    from vllm_musa_amd.fused_moe import fused_experts_impl
    w13, w2 = weights if weights is not None else synthetic.moe_bf16_weights(C2_E, C2_H, C2_I, 4000)
    x = synthetic.activations(t, C2_H, 4001 + t)
    logits = synthetic.router_logits(t, C2_E, 4002 + t, hot=8 if skewed else 0)

    def step():
        w, ids, _ = fused_topk(x, logits, TOPK, True)
        return fused_experts_impl(x, w13, w2, w, ids)
    return step, x, logits, (w13, w2)


def profile_bf16(torch, t: int, warmup: int, steps: int, log) -> int:
    step, _, _, _ = bf16_layer(torch, t)
    flush_buf = torch.ones(1 << 28, dtype=torch.int32, device="cuda")
    for _ in range(warmup):
        step()
    for _ in range(steps):
        flush_buf.max()
        torch.cuda.synchronize()
        step()
    torch.cuda.synchronize()
    a = torch.randn(4096, 4096, device="cuda").to(torch.bfloat16)
    b = torch.randn(4096, 4096, device="cuda").to(torch.bfloat16)
    for _ in range(3):
        a @ b
    torch.cuda.synchronize()
    log(f"bench: bf16 profile run done ({steps} steps at T={t}, 3 calibration matmuls)")
    return 0


# rocprofv3 counter summary of the bf16 grouped GEMMs at T=8192
# ("mfma_util_bf16_w13:" / "mfma_util_bf16_w2:" lines: MFMA busy fractions).
BF16_MFMA_SUMMARY = os.path.join("profiles", "moe_bf16_c2_mfma_and_trace.md")


def bf16_kernels(torch, x, w13, w2, logits, iters: int, flush) -> dict:
    """The bf16 layer's two grouped GEMMs at this T, each timed alone with HIP
    events on its launch stream (MoeStages), with their bf16-MFMA rooflines:
    useful flops / time against the 2.5 PF dense bf16 peak, and the MFMA busy
    fraction from the committed counter summary."""
    from vllm_musa_amd import fused_topk
    from vllm_musa_amd.fused_moe import MoeStages
    t = x.shape[0]
    w, ids, _ = fused_topk(x, logits, TOPK, True)
    st = MoeStages(x, w13, None, w2, None, w, ids, path="auto")
    st.align()
    out = {"block_m": st.block_m}
    for name, fn, fl in (("w13", st.w13_stage, 2.0 * t * TOPK * 2 * C2_I * C2_H),
                         ("w2", st.w2_stage, 2.0 * t * TOPK * C2_H * C2_I)):
        us = median_us(torch, fn, iters, flush)
        out[name] = {"us": round(us, 1), "tflops": round(fl / (us * 1e-6) / 1e12, 1),
                     "frac_bf16_peak": round(fl / (us * 1e-6) / 1e12 / PEAK_BF16_TFLOPS, 4),
                     "mfma_util": read_summary_value(BF16_MFMA_SUMMARY, f"mfma_util_bf16_{name}", float)}
    out["mfma_source"] = BF16_MFMA_SUMMARY
    del st
    return out


C4_E, C4_H, C4_I = 128, 4096, 1536
C4_T = (1, 32, 512, 4096)


def w4_configs(torch, iters: int, flush, log) -> list:
    """w4afp8 fused MoE: routing (top-8 softmax renorm) + w4afp8_moe.  Bytes =
    touched experts' int4 weights and bf16 group scales + x in + out + logits +
    routing."""
    from vllm_musa_amd import fused_topk, synthetic, w4afp8_moe
    w13, w2, s13, s2 = synthetic.moe_w4a8_weights(C4_E, C4_H, C4_I, 5000)
    per_expert = 3 * C4_I * C4_H // 2 + 2 * 3 * C4_I * (C4_H // 128)
    out = []
    for t in C4_T:
        x = synthetic.activations(t, C4_H, 5001 + t)
        logits = synthetic.router_logits(t, C4_E, 5002 + t)

        def step():
            w, ids, _ = fused_topk(x, logits, TOPK, True)
            return w4afp8_moe(x, w13, w2, s13, s2, w, ids)
        _, ids, _ = fused_topk(x, logits, TOPK, True)
        u = int(torch.unique(ids).numel())
        fl = 2.0 * t * TOPK * 3 * C4_H * C4_I
        by = u * per_expert + 4.0 * t * C4_H + 4.0 * t * C4_E + 8.0 * t * TOPK
        row = {"T": t, "experts_touched": u,
               **point(median_us(torch, step, iters, flush), fl, by, PEAK_FP8_TFLOPS)}
        row["graph_us"] = round(graph_median(torch, step, iters, flush) * 1e3, 1)
        out.append(row)
    log("bench: w4afp8 layer done")
    del w13, w2, s13, s2
    return out


NATIVE_SHAPES = ((256, 2048, 128, 8, (1, 8, 13)), (256, 7168, 2048, 8, (1,)))


def native_configs(torch, iters: int, flush, log) -> list:
    """The layer with the reference's native GEMV-MoE numerics (bf16 x against
    the fp8 weights, gate and up in fp32 through the SwiGLU): routing (top-k
    softmax renorm on ~N(0,1) logits) + fused_experts_impl.  On its calibrated
    decode shape (E=256, H=2048, I=128, top-8) path auto takes these numerics
    up to T=13, as the reference's S5000 table does; the DeepSeek-V3 layer is
    forced (path native_gemv, which the reference's VLLM_MUSA_FUSED_MOE_DISPATCH
    =gemv selects).  `w8a8_us`: the same call on the W8A8 decode kernels.
    Bytes = touched experts' fp8 weights and block scales + x in + out +
    logits + routing."""
    from vllm_musa_amd import fused_topk, synthetic
    from vllm_musa_amd.fused_moe import fused_experts_impl
    out = []
    for e, h, i, k, ts in NATIVE_SHAPES:
        w13, s13, w2, s2 = synthetic.moe_fp8_weights(e, h, i, 6000 + h)
        per_expert = 3 * i * h + 4 * ((2 * i + 127) // 128 * (h // 128) + (h + 127) // 128 * (i // 128))
        for t in ts:
            x = synthetic.activations(t, h, 6001 + t)
            logits = synthetic.router_logits(t, e, 6002 + t)
            path = "auto" if h == 2048 else "native_gemv"

            def step(p=path):
                w, ids, _ = fused_topk(x, logits, k, True)
                return fused_experts_impl(x, w13, w2, w, ids, use_fp8_w8a8=True, w1_scale=s13,
                                          w2_scale=s2, block_shape=[128, 128], path=p)
            _, ids, _ = fused_topk(x, logits, k, True)
            u = int(torch.unique(ids).numel())
            fl = 2.0 * t * k * 3 * h * i
            by = u * per_expert + 4.0 * t * h + 4.0 * t * e + 8.0 * t * k
            row = {"E": e, "H": h, "I": i, "topk": k, "T": t, "path": path, "experts_touched": u,
                   **point(median_us(torch, step, iters, flush), fl, by, PEAK_FP8_TFLOPS)}
            row["graph_us"] = round(graph_median(torch, step, iters, flush) * 1e3, 1)
            row["w8a8_us"] = round(median_us(torch, lambda: step("gemv"), iters, flush), 1)
            out.append(row)
        log(f"bench: native-GEMV layer E={e} H={h} done")
        del w13, s13, w2, s2
    return out


def native_sweep(torch, iters: int, log) -> int:
    flush_buf = torch.ones(1 << 28, dtype=torch.int32, device="cuda")
    for row in native_configs(torch, iters, lambda: flush_buf.max(), log):
        print(json.dumps(row), flush=True)
    return 0


def scales_sweep(torch, iters: int, log) -> int:
    """HIP-event medians of vmamd_convert_scales on checkpoint-load workloads
    (caches flushed by a 1 GiB read before each call): the e8m0 -> f32 upcast of
    every MoE block scale of DeepSeek-V3 (58 MoE layers x 256 experts x (32 x 56
    + 56 x 16) blocks) and the bf16 cast + check of one w4afp8 layer's group
    scales (E=128, H=4096, I=1536: w13 [128, 3072, 32], w2 [128, 4096, 12]).
    Bytes = elements x (source + destination element size)."""
    from vllm_musa_amd import _custom_ops as ops
    flush_buf = torch.ones(1 << 28, dtype=torch.int32, device="cuda")
    g = torch.Generator(device="cuda").manual_seed(5)
    work = []
    n = 58 * 256 * (32 * 56 + 56 * 16)
    src = torch.randint(100, 130, (n,), dtype=torch.uint8, device="cuda", generator=g)
    work.append(("e8m0->f32 DeepSeek-V3 MoE block scales", src,
                 torch.empty(n, dtype=torch.float32, device="cuda"), None))
    for name, shape in (("w13", (W4_E, 2 * W4_I, W4_H // 128)), ("w2", (W4_E, W4_H, W4_I // 128))):
        src = torch.rand(shape, device="cuda", generator=g) * 0.01 + 0.001
        work.append((f"f32->bf16+check w4afp8 {name} scales {list(shape)}", src,
                     torch.empty(shape, dtype=torch.bfloat16, device="cuda"),
                     torch.zeros(1, dtype=torch.int32, device="cuda")))
    for name, src, dst, bad in work:
        f = lambda: ops.convert_scales(src, dst, bad)
        for _ in range(3):
            f()
        torch.cuda.synchronize()
        us = statistics.median(time_events(torch, f, iters, lambda: flush_buf.max())) * 1e3
        by = src.numel() * (src.element_size() + dst.element_size())
        print(json.dumps({"workload": name, "elements": src.numel(), "us": round(us, 1),
                          "GBps": round(by / (us * 1e-6) / 1e9, 1),
                          "frac_hbm": round(by / (us * 1e-6) / (PEAK_HBM_GBS * 1e9), 3)}),
              flush=True)
    log("bench: checkpoint scale conversion sweep done")
    return 0


def ceiling_sweep(torch, iters: int, log) -> int:
    """The platform's own GEMMs at the dense benchmark shapes, beside this
    package's block-fp8 GEMM: torch._scaled_mm in fp8 (e4m3fn operands, bf16
    out) with one scale per tensor and, where the installed hipBLASLt takes
    them, one scale per row of A and per column of B; and torch.matmul in
    bf16.  Neither platform GEMM applies 128 x 128 block scales, so they bound
    from above what an fp8 GEMM of this shape reaches on this GPU.  HIP-event
    medians, caches flushed by a 1 GiB read before each call."""
    from vllm_musa_amd import per_token_group_quant_fp8, synthetic
    from vllm_musa_amd.block_fp8 import w8a8_block_fp8_matmul
    flush_buf = torch.ones(1 << 28, dtype=torch.int32, device="cuda")
    flush = lambda: flush_buf.max()
    fp8 = torch.float8_e4m3fn
    for n, k in C1_SHAPES:
        w, ws = synthetic.dense_fp8_weight(n, k, 7)
        for m in (512, 4096):
            x = synthetic.activations(m, k, 8)
            q, s = per_token_group_quant_fp8(x, 128)
            fl = 2.0 * m * n * k
            row = {"N": n, "K": k, "M": m}

            def rec(name, fn):
                try:
                    us = median_us(torch, fn, iters, flush)
                except RuntimeError as exc:  # a scaling mode this hipBLASLt does not take
                    row[name] = {"error": str(exc).splitlines()[0][:120]}
                    return
                row[name] = {"us": round(us, 1),
                             "frac_fp8_peak": round(fl / (us * 1e-6) / (PEAK_FP8_TFLOPS * 1e12), 3)}

            rec("block_fp8_gemm", lambda: w8a8_block_fp8_matmul(q, w, s, ws, [128, 128]))
            one = torch.ones((), dtype=torch.float32, device="cuda")
            rec("scaled_mm_tensorwise", lambda: torch._scaled_mm(q, w.t(), one, one, out_dtype=torch.bfloat16))
            sa = torch.rand(m, 1, dtype=torch.float32, device="cuda") + 0.5
            sb = torch.rand(1, n, dtype=torch.float32, device="cuda") + 0.5
            rec("scaled_mm_rowwise", lambda: torch._scaled_mm(q, w.t(), sa, sb, out_dtype=torch.bfloat16))
            xb = x.to(torch.bfloat16)
            wb = w.to(torch.bfloat16)
            rec("bf16_matmul", lambda: torch.nn.functional.linear(xb, wb))
            if "us" in row["bf16_matmul"]:
                row["bf16_matmul"]["frac_bf16_peak"] = round(
                    fl / (row["bf16_matmul"]["us"] * 1e-6) / (PEAK_BF16_TFLOPS * 1e12), 3)
            print(json.dumps(row), flush=True)
            del q, s, x, xb, wb
        del w, ws
        torch.cuda.empty_cache()
    log("bench: platform GEMM ceiling done")
    return 0


def router_sweep(torch, iters: int, log) -> int:
    """The fp32 router gate of Nemotron-H (x [M, 2688] bf16 . W [128, 2688]^T fp32)
    at M = 1, 7, 115, 512: vmamd_router_gate_fp32 against the platform's fp32
    GEMM on the same operands (F.linear(x.float(), W), the caller's own path),
    eager and as HIP-graph replays, caches flushed by a 1 GiB read before each
    call.  Bytes = W + x + logits."""
    import torch.nn.functional as F
    from vllm_musa_amd import _custom_ops as ops
    k, e = 2688, 128
    flush_buf = torch.ones(1 << 28, dtype=torch.int32, device="cuda")
    flush = lambda: flush_buf.max()
    g = torch.Generator(device="cuda").manual_seed(11)
    w = torch.randn((e, k), device="cuda", generator=g)
    for m in (1, 7, 115, 512):
        x = torch.randn((m, k), device="cuda", generator=g).to(torch.bfloat16)
        out = torch.empty((m, e), device="cuda")
        ours = lambda: ops.router_gate_fp32(x, w, out)
        plat = lambda: F.linear(x.float(), w)
        for _ in range(3):
            ours(), plat()
        torch.cuda.synchronize()
        t_ours = statistics.median(time_events(torch, ours, iters, flush)) * 1e3
        t_plat = statistics.median(time_events(torch, plat, iters, flush)) * 1e3
        g_ours = graph_median(torch, ours, iters, flush) * 1e3
        g_plat = graph_median(torch, plat, iters, flush) * 1e3
        by = e * k * 4 + m * k * 2 + m * e * 4
        print(json.dumps({"M": m, "us": round(t_ours, 2), "graph_us": round(g_ours, 2),
                          "platform_fp32_us": round(t_plat, 2),
                          "platform_fp32_graph_us": round(g_plat, 2),
                          "speedup_graph": round(g_plat / g_ours, 2),
                          "frac_hbm_graph": round(by / (g_ours * 1e-6) / (PEAK_HBM_GBS * 1e9), 3),
                          "gflops_graph": round(2.0 * m * k * e / (g_ours * 1e-6) / 1e9, 1)}),
              flush=True)
    log("bench: router gate sweep done")
    return 0


def launch_floor(torch, iters: int, log) -> int:
    """The timing floor of this file's method: n = 1, 2, 4, 8 back-to-back
    launches of a trivial kernel (an in-place add on 1024 floats), timed as
    the decode and dense points are -- HIP events around the call after an
    untimed 1 GiB read, eager and as a HIP-graph replay.  One JSON line per
    n; what a decode layer or a small GEMM adds above these is its own time."""
    flush_buf = torch.ones(1 << 28, dtype=torch.int32, device="cuda")
    flush = lambda: flush_buf.max()
    x = torch.zeros(1024, device="cuda")
    for n in (1, 2, 4, 8):
        def step(n=n):
            for _ in range(n):
                x.add_(1.0)
        for _ in range(3):
            step()
        torch.cuda.synchronize()
        eager = statistics.median(time_events(torch, step, iters, flush)) * 1e3
        graph = graph_median(torch, step, iters, flush) * 1e3
        print(json.dumps({"kernels": n, "eager_us": round(eager, 1), "graph_us": round(graph, 1),
                          "graph_minus_eager_us": round(graph - eager, 1)}), flush=True)
    log("bench: launch floor done")
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--sweep-iters", type=int, default=50)
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="only launch, three times each, the large-T kernels profiled with "
                         "rocprofv3 --pmc (fp8 W13 and W2 grouped GEMMs at T=4096, the dense "
                         "GEMM at M=4096 for 7168x18432 and 24576x1536, the w4afp8 layer at "
                         "T=4096), then three 1 GiB device copies (the traffic calibration)")
    ap.add_argument("--profile-t", type=int, default=0,
                    help="only run --steps layer steps at this T (caches flushed by a 1 GiB "
                         "read before each), for rocprofv3 --kernel-trace; prints no JSON")
    ap.add_argument("--profile-bf16", type=int, default=0,
                    help="only run --steps bf16-layer steps (E=128, top-8, H=2048, I=768) at this "
                         "T (caches flushed by a 1 GiB read before each), then three 4096^3 bf16 "
                         "matmuls (the MFMA counter calibration), for rocprofv3; prints no JSON")
    ap.add_argument("--dense", action="store_true",
                    help="only time the dense w8a8 block-fp8 GEMM / GEMV at the DeepSeek-V3 "
                         "linear shapes (one JSON line per shape)")
    ap.add_argument("--w4", action="store_true",
                    help="only time the w4afp8 MoE layer (E=128, top-8, H=4096, I=1536) at "
                         "T = 1, 32, 512, 4096 (one JSON line per T)")
    ap.add_argument("--swiglu", action="store_true",
                    help="only time the clamp-aware SwiGLU + block-fp8 down projection at the "
                         "DeepSeek-V3 dense-MLP and shared-expert shapes (one JSON line per shape)")
    ap.add_argument("--fold", action="store_true",
                    help="only time the headline layer with one shared expert, folded into the "
                         "grouped GEMMs (E+1 experts, top-8 + 1) vs run as separate dense "
                         "GEMMs, at T = 1, 16, 256, 4096 (one JSON line per T)")
    ap.add_argument("--scales", action="store_true",
                    help="only time the checkpoint scale conversions (e8m0 -> f32 of the "
                         "DeepSeek-V3 MoE block scales, f32 -> bf16 + check of a w4afp8 layer's "
                         "group scales), one JSON line per workload")
    ap.add_argument("--native", action="store_true",
                    help="only time the layer with the reference's native GEMV numerics at its "
                         "decode shapes (one JSON line per point)")
    ap.add_argument("--ceiling", action="store_true",
                    help="only time the platform's fp8 (torch._scaled_mm) and bf16 GEMMs beside "
                         "the block-fp8 GEMM at the dense benchmark shapes, M = 512 and 4096")
    ap.add_argument("--launch-floor", action="store_true",
                    help="only time 1, 2, 4 and 8 trivial kernel launches eager and as a graph "
                         "replay, by the method of the decode and dense points (one JSON line each)")
    ap.add_argument("--router", action="store_true",
                    help="only time the fp32 router gate (Nemotron-H, [M, 2688] x [128, 2688]^T) "
                         "against the platform fp32 GEMM at M = 1, 7, 115, 512")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the MoE layer runs on a single MI355X here "
              f"(--gpus {args.gpus} is not supported)", file=sys.stderr)
        return 2

    import torch

    import vllm_musa_amd
    from vllm_musa_amd import synthetic
    from vllm_musa_amd.fused_moe import Fp8MoeStages
    vllm_musa_amd.load()
    torch.cuda.set_device(0)
    log = lambda *a: print(*a, file=sys.stderr, flush=True)

    if args.dense:
        return dense_sweep(torch, args.sweep_iters, log)
    if args.w4:
        return w4_sweep(torch, args.sweep_iters, log)
    if args.swiglu:
        return swiglu_sweep(torch, args.sweep_iters, log)
    if args.scales:
        return scales_sweep(torch, args.sweep_iters, log)
    if args.router:
        return router_sweep(torch, args.sweep_iters, log)
    if args.ceiling:
        return ceiling_sweep(torch, args.sweep_iters, log)
    if args.launch_floor:
        return launch_floor(torch, args.sweep_iters, log)
    if args.native:
        return native_sweep(torch, args.sweep_iters, log)
    if args.profile_bf16 > 0:
        return profile_bf16(torch, args.profile_bf16, args.warmup, args.steps, log)

    log(f"bench: building E={E} H={H} I={I} fp8 expert stack")
    weights = synthetic.moe_fp8_weights(E, H, I, WEIGHT_SEED)
    torch.cuda.synchronize()

    if args.fold:
        return fold_sweep(torch, weights, args.sweep_iters, log)

    if args.traffic_probe:
        layer = Layer(torch, T_HEADLINE, weights)
        w, ids = layer.route()
        st = Fp8MoeStages(layer.x, *weights, w, ids, path="auto")
        st.quant()
        st.align()
        for _ in range(3):
            st.w13_stage()
        for _ in range(3):
            st.w2_stage()
        torch.cuda.synchronize()
        del st, layer, weights
        torch.cuda.empty_cache()
        from vllm_musa_amd import fused_topk, per_token_group_quant_fp8, w4afp8_moe
        from vllm_musa_amd.block_fp8 import w8a8_block_fp8_matmul
        for n, k in ((7168, 18432), (24576, 1536)):
            wd, wsd = synthetic.dense_fp8_weight(n, k, 7)
            q, s = per_token_group_quant_fp8(synthetic.activations(4096, k, 8), 128)
            for _ in range(3):
                w8a8_block_fp8_matmul(q, wd, s, wsd, [128, 128])
            torch.cuda.synchronize()
            del wd, wsd, q, s
        w4 = synthetic.moe_w4a8_weights(C4_E, C4_H, C4_I, 5000)
        x4 = synthetic.activations(4096, C4_H, 5001 + 4096)
        w, ids, _ = fused_topk(x4, synthetic.router_logits(4096, C4_E, 5002 + 4096), TOPK, True)
        for _ in range(3):
            w4afp8_moe(x4, w4[0], w4[1], w4[2], w4[3], w, ids)
        torch.cuda.synchronize()
        del w4, x4
        torch.cuda.empty_cache()
        # Calibration: a plain 1 GiB device copy whose source was evicted from
        # the caches by reading another 1 GiB first.
        src = torch.ones(1 << 30, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        other = torch.ones(1 << 28, dtype=torch.int32, device="cuda")
        for _ in range(3):
            other.max()
            dst.copy_(src)
        torch.cuda.synchronize()
        log("bench: traffic probe done (3 launches of each kernel, 3 x 1 GiB copies)")
        return 0

    if args.profile_t > 0:
        layer = Layer(torch, args.profile_t, weights)
        flush_buf = torch.ones(1 << 28, dtype=torch.int32, device="cuda")
        for _ in range(args.warmup):
            layer.step()
        for _ in range(args.steps):
            flush_buf.max()
            torch.cuda.synchronize()
            layer.step()
        torch.cuda.synchronize()
        log(f"bench: profile run done ({args.steps} steps at T={args.profile_t})")
        return 0

    # ---------------------------------------------------------- headline --
    layer = Layer(torch, T_HEADLINE, weights)
    u_head = layer.used_experts()
    for _ in range(args.warmup):
        layer.step()
    torch.cuda.synchronize()
    log(f"bench: timing {args.steps} steps at T={T_HEADLINE}")
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    w0 = time.perf_counter()
    ev0.record()
    for _ in range(args.steps):
        layer.step()
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - w0
    ms = ev0.elapsed_time(ev1) / args.steps
    flops = layer_flops(T_HEADLINE * TOPK)
    value = flops / (ms * 1e-3) / 1e12
    head_bytes = layer_bytes(T_HEADLINE, u_head)

    # --------------------------------------------- dominant kernel: W13 ----
    w, ids = layer.route()
    st = Fp8MoeStages(layer.x, *weights, w, ids, path="auto")
    st.quant()
    st.align()
    for _ in range(3):
        st.w13_stage()
    torch.cuda.synchronize()
    k_ms = statistics.mean(time_events(torch, st.w13_stage, max(args.steps, 10)))
    k_bytes = w13_bytes(T_HEADLINE, u_head)
    k_gbs = k_bytes / (k_ms * 1e-3) / 1e9
    roofline = {"bound": "hbm", "achieved": round(k_gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(k_gbs / PEAK_HBM_GBS, 4), "traffic": read_traffic(),
                "traffic_source": TRAFFIC_SUMMARY,
                "kernel": "moe_big_kernel<W13>" if st.block_m == 256 else "moe_gemm_dma_kernel<kFp8, W13>",
                "kernel_us": round(k_ms * 1e3, 1),
                "kernel_tflops": round(2.0 * T_HEADLINE * TOPK * 2 * I * H / (k_ms * 1e-3) / 1e12, 1),
                "algorithmic_bytes": int(k_bytes),
                "mfma_util": read_summary_value(MFMA_SUMMARY, "mfma_util_w13", float),
                "mfma_source": MFMA_SUMMARY}
    del st

    # ------------------------------------------------------------- sweep ---
    sweep = []
    if not args.no_sweep:
        # Untimed cache flush before each call: reading 1 GiB evicts the L2s
        # and the 256 MB memory-side cache without leaving dirty lines (after
        # a 1 GiB fill the timed kernels would pay for writing those back; in
        # a model the kernels ahead of a MoE layer mostly read weights).
        flush_buf = torch.ones(1 << 28, dtype=torch.int32, device="cuda")
        flush = lambda: flush_buf.max()
        for t in SWEEP_T:
            lay = layer if t == T_HEADLINE else Layer(torch, t, weights)
            u = lay.used_experts()
            med = median_us(torch, lay.step, args.sweep_iters, flush) * 1e-3
            gmed = graph_median(torch, lay.step, args.sweep_iters, flush)
            f = layer_flops(t * TOPK)
            b = layer_bytes(t, u)
            ideal = max(f / (PEAK_FP8_TFLOPS * 1e12), b / (PEAK_HBM_GBS * 1e9))
            sweep.append({"T": t, "experts_touched": u, "us": round(med * 1e3, 1),
                          "tflops": round(f / (med * 1e-3) / 1e12, 2),
                          "gbps": round(b / (med * 1e-3) / 1e9, 1),
                          "frac_hbm": round(b / (med * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                          "frac_fp8_peak": round(f / (med * 1e-3) / 1e12 / PEAK_FP8_TFLOPS, 4),
                          "frac_roofline": round(ideal / (med * 1e-3), 4),
                          "graph_us": round(gmed * 1e3, 1),
                          "graph_frac_roofline": round(ideal / (gmed * 1e-3), 4)})
            log(f"bench: sweep {sweep[-1]}")
        del flush_buf

    # ---------------------------------- the metric's other configurations --
    extra = {}
    if not args.no_sweep:
        flush_buf = torch.ones(1 << 28, dtype=torch.int32, device="cuda")
        flush = lambda: flush_buf.max()
        extra["dense"] = dense_configs(torch, args.sweep_iters, flush, log)
        extra["bf16_moe"] = bf16_configs(torch, args.sweep_iters, flush, log)
        extra["w4afp8_moe"] = w4_configs(torch, args.sweep_iters, flush, log)
        extra["native_gemv"] = native_configs(torch, args.sweep_iters, flush, log)
        del flush_buf

    cpu = None
    if not args.no_cpu:
        log("bench: CPU baseline (bounded sample)")
        cpu = cpu_baseline(torch, layer)

    line = {
        "metric": METRIC, "value": round(value, 2), "unit": "TFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "wall_s_timed": round(wall, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp8", "data": "synthetic",
        "config": {"workload": "DeepSeek-V3-shape fp8 block MoE layer (routing + fused experts)",
                   "T": T_HEADLINE, "E": E, "topk": TOPK, "H": H, "I": I,
                   "routing": "grouped sigmoid+bias, 8 groups / top-4, renorm, x2.5",
                   "weights": "e4m3fn, 128x128 block scales", "activations": "1x128 fp8 groups",
                   "experts_touched": u_head, "algorithmic_gbps":
                       round(head_bytes / (ms * 1e-3) / 1e9, 1)},
        "roofline": roofline, "cpu_baseline": cpu, "sweep": sweep, **extra,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
