"""exl3xpu: EXL3 routed-expert offload for MI355X (HIP kernels behind the reference's exl3xpu_moe op schemas).

moe_offload  -- ops() loader, planar4 / pack_expert, ExpertStore (HBM slot cache + pinned host arena)
nvtier       -- TierStore, NvTier / NvTierFast / NvTierAsync (RAM tier with admission control)
capi         -- ctypes binding of the C-ABI library libexl3moe.so (include/exl3moe.h)
synth        -- seeded synthetic experts and routing traces
"""
