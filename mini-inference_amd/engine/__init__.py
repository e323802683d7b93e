"""Host-side mirror of mini-inference's engine packages that sit on the quantized path.

Only `engine.quantization` (quantized linears and experts) and `engine.core.kv_cache`
(8-bit KV formats) are provided; the serving engine around them is out of scope.
"""
