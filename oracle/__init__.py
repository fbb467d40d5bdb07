"""CPU oracle of the quantized fused-MoE / block-fp8 matmul path.

TEST INFRASTRUCTURE ONLY.  This package restates, in plain numpy, the
algorithms of MooreThreads/vllm-musa for this path (each function cites the
reference file:line it follows).  It is imported only by ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``, and
there only as the checker (or as the timed CPU baseline) -- never as the thing
measured on the GPU and never as a fallback of the product path, which lives in
``vllm-musa_amd/`` and fails loudly when its HIP library is missing.

Modules:
  numerics  -- bit-exact e4m3fn / bf16 encoders and decoders
  quant     -- 1x128 group quantiser, SiLU-and-mul (+quant)
  routing   -- softmax / sigmoid top-k, grouped top-k
  align     -- moe_align_block_size (stable counting sort with padding)
  gemm      -- w8a8 block-fp8 GEMM (fp64 closed form)
  moe       -- fused experts (bf16 and fp8-block), moe_sum
  w4afp8    -- the w4afp8 MoE reference
  scales    -- checkpoint scale conversion (e8m0 upcast, bf16 cast + check)
  router_gate -- fp32 router-gate GEMM in its fixed summation order

How each function is pinned (golden vectors, closed forms, brute force,
library cross-checks) is listed in tests/test_oracle_*.py.
"""
