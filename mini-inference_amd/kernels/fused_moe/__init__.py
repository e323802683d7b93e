"""Fused INT4 / INT8 MoE: HIP moe_align + grouped weight-only expert GEMMs."""
from kernels.fused_moe.moe_int4 import fused_moe_int4, fused_moe_int8, moe_align  # noqa: F401
