"""Fused INT4 / INT8 / FP8 MoE: HIP moe_align + grouped expert GEMMs."""
from kernels.fused_moe.moe_int4 import fused_moe_fp8, fused_moe_int4, fused_moe_int8, moe_align  # noqa: F401
