"""Split-KV paged decode attention on bf16 / fp8 / int8 KV caches (HIP, gfx950)."""
from kernels.paged_attention.decode import choose_partition, paged_decode_attention  # noqa: F401
