"""CPU oracle for the EXL3 expert-offload hot path.

TEST INFRASTRUCTURE ONLY. Nothing in the product (the `exl3xpu` package, its HIP kernels or its C-ABI library)
imports, links or calls anything in this directory. Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline`
leg of `bench.py` use it, and only as the checker / the timed CPU restatement.

Modules:
  exl3      -- EXL3 mul1 codebook, trellis tile decode, PLANAR4 packing, blob layout, fwht128, expert forward
               (decode and prefill rounding points), token alignment.
  synth     -- seeded synthetic weights, routing and Zipf decode traces.
  cache     -- canonical device-cache `ensure` + host admission step (ctypes wrapper of cache_oracle.c).
  cpu_path  -- the PyTorch CPU restatement timed as the CPU baseline.

Every function cites the reference file:line it restates. Parity-pinning status per function is listed in the
header of each module.
"""
