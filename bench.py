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
K timed steps; `sweep` gives us / TFLOP/s / GB/s and roofline fractions at
T = 1, 16, 256, 4096 (cold weights: a 1 GiB buffer is read between
iterations; `graph_us` is the same step replayed from a HIP graph, as a
serving engine runs decode); `roofline` is the dominant kernel (W13 grouped
GEMM at T=4096) timed on its own with HIP events on its launch stream, its
`traffic` (HBM bytes per launch) read from the committed rocprofv3 counter
summary; `cpu_baseline` times the CPU oracle on a bounded sample of the same
layer.

  python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-sweep] [--no-cpu]
  python bench.py --traffic-probe   # the launches profiled for FETCH_SIZE / WRITE_SIZE
  python bench.py --dense           # dense block-fp8 linear shapes, M = 1 .. 4096 (JSON lines)
  python bench.py --w4              # w4afp8 MoE layer, T = 1 .. 1024 (JSON lines)
  python bench.py --swiglu          # clamped SwiGLU + block-fp8 down projection (JSON lines)
  python bench.py --fold            # shared expert folded into the MoE vs run as dense GEMMs
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

# MI355X published peaks.
PEAK_HBM_GBS = 8000.0
PEAK_FP8_TFLOPS = 5000.0

E, H, I, TOPK, GROUPS, TOPK_GROUP, SCALE = 256, 7168, 2048, 8, 8, 4, 2.5
T_HEADLINE = 4096
SWEEP_T = (1, 16, 256, 4096)
WEIGHT_SEED = 3000

METRIC = "fp8-block MoE layer µs, TFLOPS & HBM GB/s (% roofline) at T=1..4096"

# rocprofv3 counter summary of the W13 kernel at T=4096 (FETCH_SIZE and
# WRITE_SIZE per dispatch, scaled by a 1 GiB copy); its
# "traffic_bytes_per_launch:" line fills roofline.traffic.
TRAFFIC_SUMMARY = os.path.join("profiles", "moe_w13_gemm_fp8_dsv3_T4096_traffic.md")


def read_traffic() -> int | None:
    path = os.path.join(ROOT, TRAFFIC_SUMMARY)
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            return int(line.split(":", 1)[1].strip())
    return None


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


def cpu_baseline(torch, layer: Layer, target_s: float = 15.0) -> dict:
    """Time the CPU oracle on a bounded sample of the T=4096 layer: the routes
    of a few experts (their tokens, their weights), same arithmetic as the
    full layer.  Reported in the layer's unit (TFLOP/s)."""
    import numpy as np

    from oracle import moe as omoe
    try:
        from threadpoolctl import threadpool_info
        threads = max([d.get("num_threads", 1) for d in threadpool_info()] or [1])
    except Exception:  # pragma: no cover
        threads = 1
    w, ids = layer.route()
    ids_np = ids.cpu().numpy()
    w_np = w.cpu().numpy()
    x_np = layer.x.float().cpu().numpy()
    counts = np.bincount(ids_np.ravel(), minlength=E)
    order = np.argsort(-counts, kind="stable")
    done_routes, elapsed, n_exp = 0, 0.0, 0
    for e in order:
        if elapsed >= target_s or n_exp >= 16:
            break
        toks = np.nonzero((ids_np == e).any(axis=1))[0]
        sub_ids = np.where(ids_np[toks] == e, 0, -1).astype(np.int32)
        sel = torch.tensor([int(e)], device=layer.w13.device)
        u8 = lambda t: t.view(torch.uint8).index_select(0, sel).cpu().numpy()
        f32 = lambda t: t.index_select(0, sel).cpu().numpy()
        args = (x_np[toks], u8(layer.w13), f32(layer.s13), u8(layer.w2), f32(layer.s2),
                w_np[toks], sub_ids)
        t0 = time.perf_counter()
        omoe.fused_experts_fp8(*args)
        elapsed += time.perf_counter() - t0
        done_routes += int((sub_ids >= 0).sum())
        n_exp += 1
    tflops = layer_flops(done_routes) / elapsed / 1e12
    return {"value": round(tflops, 6), "unit": "TFLOP/s", "cores": int(threads), "kind": "port",
            "sample": f"numpy float64 oracle (oracle/moe.py fused_experts_fp8) on {n_exp} experts of "
                      f"the T={layer.t} layer ({done_routes} routes, {elapsed:.1f} s); full-layer "
                      f"CPU time extrapolates to "
                      f"{layer_flops(layer.t * TOPK) / (tflops * 1e12):.0f} s"}


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
    """HIP-event medians of routing + w4afp8_moe (caches flushed by a 1 GiB read
    before each call); bytes = touched experts' int4 weights and bf16 scales +
    activations + output."""
    from vllm_musa_amd import fused_topk, synthetic, w4afp8_moe
    w13, w2, s13, s2 = synthetic.moe_w4a8_weights(W4_E, W4_H, W4_I, 12)
    flush_buf = torch.ones(1 << 28, dtype=torch.int32, device="cuda")
    per_expert = 3 * W4_I * W4_H // 2 + 2 * 3 * W4_I * (W4_H // 128)
    for t in (1, 16, 256, 1024):
        x = synthetic.activations(t, W4_H, 100 + t)
        logits = synthetic.router_logits(t, W4_E, 200 + t)
        def f():
            w, ids, _ = fused_topk(x, logits, TOPK, True)
            return w4afp8_moe(x, w13, w2, s13, s2, w, ids)
        for _ in range(3):
            f()
        torch.cuda.synchronize()
        _, ids, _ = fused_topk(x, logits, TOPK, True)
        used = int(torch.unique(ids).numel())
        us = statistics.median(time_events(torch, f, iters, lambda: flush_buf.max())) * 1e3
        by = used * per_expert + 2 * t * W4_H * 2
        fl = 2.0 * t * TOPK * 3 * W4_H * W4_I
        print(json.dumps({"T": t, "experts_touched": used, "us": round(us, 1),
                          "frac_hbm": round(by / (us * 1e-6) / (PEAK_HBM_GBS * 1e9), 3),
                          "tflops": round(fl / (us * 1e-6) / 1e12, 2)}), flush=True)
    log("bench: w4afp8 sweep done")
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


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--sweep-iters", type=int, default=20)
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="only launch the W13 kernel at T=4096 three times, then three "
                         "1 GiB device copies (the counter calibration), for rocprofv3 --pmc")
    ap.add_argument("--profile-t", type=int, default=0,
                    help="only run --steps layer steps at this T (caches flushed by a 1 GiB "
                         "read before each), for rocprofv3 --kernel-trace; prints no JSON")
    ap.add_argument("--dense", action="store_true",
                    help="only time the dense w8a8 block-fp8 GEMM / GEMV at the DeepSeek-V3 "
                         "linear shapes (one JSON line per shape)")
    ap.add_argument("--w4", action="store_true",
                    help="only time the w4afp8 MoE layer (E=128, top-8, H=4096, I=1536) at "
                         "T = 1, 16, 256, 1024 (one JSON line per T)")
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
        torch.cuda.synchronize()
        del st, layer, weights
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
        log("bench: traffic probe done (3 W13 launches, 3 x 1 GiB copies)")
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
                "kernel": "moe_gemm_dma_kernel<kFp8, W13>",
                "kernel_us": round(k_ms * 1e3, 1),
                "kernel_tflops": round(2.0 * T_HEADLINE * TOPK * 2 * I * H / (k_ms * 1e-3) / 1e12, 1),
                "algorithmic_bytes": int(k_bytes)}
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
            for _ in range(3):
                lay.step()
            torch.cuda.synchronize()
            times = time_events(torch, lay.step, args.sweep_iters, flush)
            med = statistics.median(times)
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
        "roofline": roofline, "cpu_baseline": cpu, "sweep": sweep,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
