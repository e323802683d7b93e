"""Fused INT4 MoE: HIP moe_align + grouped W4A16 expert GEMMs."""
from kernels.fused_moe.moe_int4 import fused_moe_int4, moe_align  # noqa: F401
