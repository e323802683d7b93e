"""CPU oracle for the quantized path: TEST INFRASTRUCTURE ONLY.

A plain PyTorch-on-CPU (and numpy) restatement of the reference's formulas, each
function citing the reference file:line it follows. Only tests/, the smoke check of
__graft_entry__ and the `cpu_baseline` leg of bench.py may import it, and only as the
checker or the timed CPU baseline; the product path (mini-inference_amd/) never calls it.

Modules:
  quant     int8 / int4 / fp8 quantize, dequantize, linear; KV quantize-on-write
  attention paged decode attention (fp32 per-request loop)
  moe       moe_align, per-expert INT4 MoE reference
  codecs    independent numpy codecs (bf16 RNE, e4m3fn table) that pin torch's casts

Pinning (what checks each function, see tests/test_oracle.py):
  * codecs are checked against closed forms of the formats and brute force;
  * torch's bf16 / e4m3fn casts used by `quant` are checked against `codecs`;
  * quant: hand-derived known answers in tests/golden/known_answers.json, exact
    round trips and the reference's own error bounds (tests/test_quantizaton.py:14-16);
  * attention: a float64 numpy softmax, closed forms (one token, equal keys), split /
    page-size invariance, GQA == repeated kv heads;
  * moe: invariants of tests/test_fused_moe.py:39-53 and a dense single-expert closed form.
"""
