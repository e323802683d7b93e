"""gfx950 kernels of the quantized path (libmiq.so) and their torch-facing wrappers."""
