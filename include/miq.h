/* libmiq: MI355X (gfx950) kernels for mini-inference's quantized compute path.
 *
 * C ABI only: raw device pointers, element counts/strides in elements (int64), a dtype
 * enum for operands whose type varies, and the HIP stream to launch on (passed as
 * void* so this header needs no HIP include). No function allocates device memory or
 * keeps state between calls, and only miq_device_errors synchronises the host. The one
 * exception to "no state": the split-K counters and exchange words inside a
 * caller-provided workspace are left at zero by every call (the caller zeroes the
 * workspace once when it allocates it).
 *
 * Every function returns MIQ_OK (0) or a negative MIQ_ERR_* code; miq_last_error()
 * returns a thread-local message for the last failure.
 *
 * Reference citations are paths in davidjoyme/mini-inference.
 */
#ifndef MIQ_H_
#define MIQ_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum miq_status {
  MIQ_OK = 0,
  MIQ_ERR_INVALID = -1,  /* bad shape / dtype / alignment argument */
  MIQ_ERR_LAUNCH = -2,   /* the HIP launch failed */
};

enum miq_dtype {
  MIQ_F32 = 0,
  MIQ_BF16 = 1,
  MIQ_F16 = 2,
  MIQ_FP8_E4M3 = 3, /* OCP e4m3fn, torch.float8_e4m3fn */
  MIQ_INT8 = 4,
  MIQ_UINT8 = 5,
  MIQ_INT32 = 6,
  MIQ_INT64 = 7,
};

const char* miq_last_error(void);
int miq_abi_version(void);

/* Device-side failures that a kernel cannot return as a status: bits of a per-GPU error
 * word that kernels set and miq_device_errors() reads. No counterpart in the reference
 * (its kernels have no bounded waits). */
enum miq_device_error {
  MIQ_DEVERR_PANEL_WAIT = 1, /* the INT4 panel GEMM's split-K reducer gave up waiting for a
                                partial; the affected outputs were written as NaN */
};

/* Waits for `stream`, stores the current device's error word in *bits and clears it.
 * A diagnostic for tests and health checks: it synchronises, unlike every other entry
 * point. No counterpart in the reference. */
int miq_device_errors(unsigned* bits, void* stream);

/* Text for error word `bits` (host only, needs no GPU). */
const char* miq_device_error_string(unsigned bits);

/* Reads `bytes` bytes (a multiple of 16) of `buf` as a plain stream: the HBM streaming
 * floor a benchmark sets kernel times against. No counterpart in the reference (a
 * measurement helper); `sink` is a device int that is practically never written. */
int miq_stream_read(const void* buf, size_t bytes, int* sink, void* stream);

/* Re-reads the MIQ_* kernel-selection variables (MIQ_WO_STREAM, MIQ_WO_PANEL, ...), which
 * the library otherwise reads once when it is loaded. No counterpart in the reference: a
 * hook for tests and tuning runs that switch kernels inside one process. Not to be
 * called while another thread launches kernels of this library. */
int miq_tuning_reload(void);

/* ------------------------------------------------------------------ weight quantization
 * Replaces Int8WeightOnly.quantize (engine/quantization/int8_wo.py:8-12):
 *   s = max|w_row| clamped to 1e-8, divided by 127 (fp32); q = round_half_even(w / s)
 *   clamped to [-127, 127]; scale stored as bf16(s) / f16(s) / s per scale_dtype.
 * w: [rows, K] (w_dtype bf16/f16/f32, row stride ldw), q: int8 [rows, K] contiguous,
 * scale: [rows] of scale_dtype. */
int miq_int8_quantize(const void* w, int w_dtype, int64_t rows, int64_t K, int64_t ldw,
                      int8_t* q, void* scale, int scale_dtype, void* stream);

/* Replaces Int8WeightOnly.dequantize (int8_wo.py:14-15): out = q.to(dt) * scale in dt
 * (dt = scale_dtype, one rounding). out: [rows, K] contiguous. */
int miq_int8_dequantize(const int8_t* q, const void* scale, int scale_dtype, int64_t rows,
                        int64_t K, void* out, void* stream);

/* Replaces Int4WeightOnly.quantize (engine/quantization/int4_wo.py:15-31): per group of
 * `group` along K, s = ((max - min) / 15) clamped to 1e-8, q = round((w - min) / s)
 * clamped to [0, 15]; packed two per byte, even k in the low nibble; scale and zero
 * (= group min) stored in sz_dtype. q: [rows, K/2], scale/zero: [rows, K/group].
 * zero == NULL selects the symmetric format (no counterpart in the reference; used by the
 * benchmark's INT4 configuration): s = max|w| / 7 clamped to 1e-8,
 * code = clamp(round(w / s), -8, 7) + 8, dequantized as (code - 8) * s. */
int miq_int4_quantize(const void* w, int w_dtype, int64_t rows, int64_t K, int64_t ldw,
                      int64_t group, uint8_t* q, void* scale, void* zero, int sz_dtype,
                      void* stream);

/* Replaces Int4WeightOnly.dequantize (int4_wo.py:33-42): w = (q * scale) + zero with a
 * rounding to sz_dtype after each operation. zero == NULL selects the symmetric form
 * w = (q - 8) * scale (one rounding). out: [rows, K] in sz_dtype. */
int miq_int4_dequantize(const uint8_t* q, const void* scale, const void* zero, int sz_dtype,
                        int64_t rows, int64_t K, int64_t group, void* out, void* stream);

/* Replaces FP8WeightAct.quantize (engine/quantization/fp8.py:32-36) and
 * FP8WeightAct.quantize_activation (fp8.py:41-46), which are the same formula:
 *   s = max|x_row| clamped to 1e-12, divided by 448 (fp32);
 *   q = e4m3fn(clamp(x / s, -448, 448)).
 * x: [rows, K] (x_dtype bf16/f16/f32, row stride ldx), q: [rows, K] contiguous bytes,
 * scale: fp32 [rows]. */
int miq_fp8_quantize_rows(const void* x, int x_dtype, int64_t rows, int64_t K, int64_t ldx,
                          uint8_t* q, float* scale, void* stream);

/* Replaces FP8WeightAct.dequantize (fp8.py:38-39): out fp32 [rows, K] = q * scale[row]. */
int miq_fp8_dequantize(const uint8_t* q, const float* scale, int64_t rows, int64_t K,
                       float* out, void* stream);

/* ------------------------------------------------------------------ weight-only GEMMs
 * Any M >= 1: decode kernels up to M = 64, a dequantize-in-the-K-loop MFMA GEMM above
 * (prefill), which splits K when the output has fewer 64 x 128 tiles than CUs, and, where
 * its 128 x 128..384 tiles fill the GPU (long prefill chunks), a GEMM that dequantizes
 * each weight block once per workgroup for the bf16 MFMA.
 * Workspace for the split-K reduction of the two weight-only GEMMs and for the last
 * kernel's packed activations and K-split partials. Its first 16384 bytes hold arrival
 * counters that must be zero before the first call (zero the whole buffer once when
 * allocating it); every call leaves the whole workspace at zero again (counters, fp32
 * partials and packed activations alike). A workspace below this size for a long prefill call makes it take
 * the prefill kernel. Calls that share one workspace must be ordered (same stream). */
size_t miq_wo_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, int weight_bits);

/* Replaces Int8WeightOnly.linear (int8_wo.py:17-21):
 *   y = bf16( bf16(x @ q^T) * bf16(scale) )
 * x: bf16 [M, K] row stride ldx; q: int8 [N, K] contiguous; scale: [N] of scale_dtype;
 * y: bf16 [M, N] row stride ldy. M >= 1, K % 128 == 0, N % 16 == 0. */
int miq_w8a16_gemm(const void* x, int64_t ldx, const int8_t* q, const void* scale,
                   int scale_dtype, void* y, int64_t ldy, int64_t M, int64_t N, int64_t K,
                   void* workspace, size_t workspace_bytes, void* stream);

/* Replaces Int4WeightOnly.linear = QuantMethod.linear over Int4WeightOnly.dequantize
 * (engine/quantization/base.py:20-24, int4_wo.py:33-42): y = bf16(x @ W^T) with
 * W = q * scale + zero (zero == NULL: W = (q - 8) * scale), evaluated in fp32 as
 * scale * (x . q) + zero * sum(x) per group (the wide kernel of long prefill calls
 * multiplies W rounded once to bf16, as the reference's bf16 weights are). x: bf16 [M, K];
 * q: uint8 [N, K/2];
 * scale/zero: [N, K/group] of sz_dtype (bf16/f16/f32). M >= 1, group % 128 == 0,
 * K % group == 0, N % 16 == 0. */
int miq_w4a16_gemm(const void* x, int64_t ldx, const uint8_t* q, const void* scale,
                   const void* zero, int sz_dtype, int64_t group, void* y, int64_t ldy,
                   int64_t M, int64_t N, int64_t K, void* workspace, size_t workspace_bytes,
                   void* stream);

/* miq_w4a16_gemm without a workspace argument, for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). No counterpart in the reference. The split-K scratch is a static device array
 * of 32 MiB that each GPU holds until the process ends; shapes whose split-K scratch
 * exceeds it are rejected (MIQ_ERR_INVALID); long prefill calls whose packed activations
 * and K-split partials would not fit take the prefill kernel. Every call on a GPU shares that GPU's array: calls that
 * overlap on one GPU (two streams, two threads) race and give wrong results; calls ordered
 * on one stream are safe. Allocates nothing; the first call on a device looks up the
 * array's address there. Same arguments and results as miq_w4a16_gemm. */
int miq_w4a16_gemm_noalloc(const void* x, int64_t ldx, const uint8_t* q, const void* scale,
                           const void* zero, int sz_dtype, int64_t group, void* y, int64_t ldy,
                           int64_t M, int64_t N, int64_t K, void* stream);

/* ------------------------------------------------------------------ FP8 prefill GEMM
 * Replaces the torch._scaled_mm call of FP8WeightAct.linear (fp8.py:55-61):
 *   y[m, n] = bf16( (sum_k xq[m,k] * wq[n,k]) * x_scale[m] * w_scale[n] )
 * xq: e4m3 [M, K] contiguous, wq: e4m3 [N, K] contiguous, scales fp32, y: bf16 [M, N]
 * row stride ldy. K % 128 == 0. */
int miq_fp8_gemm(const uint8_t* xq, const float* x_scale, const uint8_t* wq,
                 const float* w_scale, void* y, int64_t ldy, int64_t M, int64_t N, int64_t K,
                 void* stream);

/* ------------------------------------------------------------------ KV cache
 * Replaces KVCache._quantize + KVCache.write (engine/core/kv_cache.py:359-388) for one
 * layer and one of K or V: per (token, head) s = bf16(clamp(max|x| / qmax, 1e-8)),
 * q = x / s (int8: round-half-even, clamp +-127; fp8: clamp +-448, e4m3fn), written to
 * row slots[t] of the cache. x: [T, heads, D] (x_dtype bf16/f16/f32, strides in
 * elements), cache: [slots, heads, D] bytes (kv_dtype MIQ_INT8 or MIQ_FP8_E4M3),
 * cache_scale: [slots, heads] of scale_dtype. slots: int64 [T]. */
int miq_kv_quant_write(const void* x, int x_dtype, int64_t T, int64_t heads, int64_t D,
                       int64_t x_stride_t, int64_t x_stride_h, const int64_t* slots,
                       void* cache, int kv_dtype, int64_t c_stride_t, int64_t c_stride_h,
                       void* cache_scale, int scale_dtype, int64_t s_stride_t,
                       int64_t s_stride_h, void* stream);

/* ------------------------------------------------------------------ paged decode attention
 * Replaces paged_decode_attention (kernels/paged_attention/decode_triton.py:123-180):
 *   out[b, h] = softmax(sm_scale * q[b,h] . K_b^T) V_b over seq_lens[b] tokens, token i
 *   of request b at cache row block_table[b, i / page] * page + i % page, kv head
 *   h / (H / KV); 8-bit caches dequantized as value * scale[row, kv head].
 * q, out: bf16 [B, H, D] (strides in elements, last dim contiguous); k/v cache
 * [slots, KV, D] with kv_dtype MIQ_BF16 / MIQ_FP8_E4M3 / MIQ_INT8 (strides in elements);
 * k_scale/v_scale: NULL or [slots, KV] of scale_dtype with strides (s_stride_t,
 * s_stride_h) (0, 0 for one per-tensor value); block_table int32 [B, max_pages] row
 * stride bt_stride, whose memory spans B * bt_stride entries (entries past a request's
 * pages may be read, not used); seq_lens int32 [B]. D == 128.
 * The context of each request is cut into partitions of `partition` tokens (multiple of
 * 128). Workspace: o_part fp32 [B, H, max_parts, D] and lse_part fp32 [B, H, max_parts],
 * max_parts >= ceil(max(seq_lens) / partition). */
int miq_paged_decode(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                     const void* k_cache, const void* v_cache, int kv_dtype,
                     int64_t kv_stride_t, int64_t kv_stride_h,
                     const void* k_scale, const void* v_scale, int scale_dtype,
                     int64_t s_stride_t, int64_t s_stride_h,
                     const int32_t* block_table, int64_t bt_stride, const int32_t* seq_lens,
                     int64_t B, int64_t H, int64_t KV, int64_t D, int64_t page,
                     float sm_scale, int64_t partition, int64_t max_parts,
                     float* o_part, float* lse_part,
                     void* out, int64_t out_stride_b, int64_t out_stride_h, void* stream);

/* ------------------------------------------------------------------ fused MoE (INT4 experts)
 * Replaces moe_align (kernels/fused_moe/csrc/moe_align.cu:5-88,
 * kernels/fused_moe/fused_moe_triton.py:8-39): groups the T*k (token, slot) pairs of
 * topk_ids by expert, each group padded to a multiple of block_m with the sentinel T*k.
 * topk_ids: [num_pairs] int32 or int64 (idx_dtype); sorted_ids int32
 * [num_pairs + E*(block_m-1)]; expert_ids int32 [ceil(that / block_m)]; num_padded int32 [1].
 * Within one expert, pairs are in ascending pair order (deterministic). */
int miq_moe_align(const void* topk_ids, int idx_dtype, int64_t num_pairs, int64_t E,
                  int64_t block_m, int32_t* sorted_ids, int32_t* expert_ids,
                  int32_t* num_padded, void* stream);

/* Replaces QuantExperts.forward (engine/quantization/modules.py:55-75) for Int4WeightOnly
 * experts: out[t] = sum_j w[t,j] * down_e( silu(gate_e(x_t)) * up_e(x_t) ), e = ids[t,j].
 * hidden: bf16 [T, H]; gate_up q: uint8 [E, 2I, H/2], scale/zero [E, 2I, H/group];
 * down q: uint8 [E, H, I/2], scale/zero [E, H, I/group]; zero pointers may be NULL
 * (symmetric); topk_weights [T, k] in w_dtype (f32 / bf16 / f16, k <= 32); sorted_ids /
 * expert_ids / num_padded from miq_moe_align with block_m == 16. Workspace bytes from
 * miq_moe_workspace_bytes. out: bf16 [T, H].
 * Rounding follows the reference loop: gate/up and down outputs rounded to bf16, the
 * product with the routing weight (in its own dtype) rounded to bf16, and a token's
 * contributions added in ascending expert order with a bf16 rounding after each
 * addition (index_add_ into a bf16 output). */
size_t miq_moe_workspace_bytes(int64_t T, int64_t topk, int64_t E, int64_t H, int64_t I);
int miq_w4a16_moe(const void* hidden, int64_t T, int64_t H, int64_t I, int64_t E, int64_t topk,
                  const uint8_t* gu_q, const void* gu_scale, const void* gu_zero,
                  const uint8_t* dn_q, const void* dn_scale, const void* dn_zero,
                  int sz_dtype, int64_t group, const void* topk_weights, int w_dtype,
                  const int32_t* sorted_ids, const int32_t* expert_ids,
                  const int32_t* num_padded, void* workspace, size_t workspace_bytes,
                  void* out, void* stream);

/* Replaces QuantExperts.forward (engine/quantization/modules.py:55-75) for Int8WeightOnly
 * experts with a SiLU gate: the same layer as miq_w4a16_moe on int8 weights.
 * gate_up q: int8 [E, 2I, H], scale [E, 2I] (or [E, 2I, 1]); down q: int8 [E, H, I],
 * scale [E, H]; scale_dtype bf16 / f16 / f32. Each expert linear is int8_wo.linear's
 * bf16(bf16(x @ q^T) * bf16(scale)) (int8_wo.py:17-21); the rest (SiLU gate, routing
 * weight, expert-ordered bf16 combine) as miq_w4a16_moe. H and I multiples of 128;
 * sorted_ids / expert_ids / num_padded from miq_moe_align with block_m == 16; workspace
 * from miq_moe_workspace_bytes. out: bf16 [T, H]. */
int miq_w8a16_moe(const void* hidden, int64_t T, int64_t H, int64_t I, int64_t E, int64_t topk,
                  const int8_t* gu_q, const void* gu_scale, const int8_t* dn_q, const void* dn_scale,
                  int scale_dtype, const void* topk_weights, int w_dtype,
                  const int32_t* sorted_ids, const int32_t* expert_ids,
                  const int32_t* num_padded, void* workspace, size_t workspace_bytes,
                  void* out, void* stream);

/* Replaces QuantExperts.forward (engine/quantization/modules.py:55-75) for FP8WeightAct
 * experts with a SiLU gate on a native-FP8 device: the same layer as miq_w4a16_moe with
 * every expert linear FP8WeightAct.linear (engine/quantization/fp8.py:41-61): activation
 * rows quantized per row to e4m3fn with s = max(amax, 1e-12) / 448, then
 * bf16(sum(x_q w_q) * s_x * s_w) as torch._scaled_mm returns it.
 * gate_up q: e4m3fn bytes [E, 2I, H], scale fp32 [E, 2I]; down q: e4m3fn bytes [E, H, I],
 * scale fp32 [E, H]. H and I multiples of 128 and at most 4096; sorted_ids / expert_ids /
 * num_padded from miq_moe_align with block_m == 16; workspace from
 * miq_moe_workspace_bytes. out: bf16 [T, H]. */
int miq_fp8_moe(const void* hidden, int64_t T, int64_t H, int64_t I, int64_t E, int64_t topk,
                const uint8_t* gu_q, const float* gu_scale, const uint8_t* dn_q, const float* dn_scale,
                const void* topk_weights, int w_dtype, const int32_t* sorted_ids,
                const int32_t* expert_ids, const int32_t* num_padded, void* workspace,
                size_t workspace_bytes, void* out, void* stream);

/* The three layers above with the routing taken straight from topk_ids ([T, k] int32 or
 * int64, idx_dtype; the reference's fused_moe call takes topk_ids and aligns them itself,
 * kernels/fused_moe/fused_moe_triton.py:110-121, moe_align.cu:5-88). Up to 1024 pairs and
 * 256 experts (and, for int4, H a multiple of 128 and I of 64) the expert GEMMs form
 * moe_align's layout in LDS and no align launch runs; otherwise miq_moe_align runs into the
 * workspace. Same results as miq_moe_align followed by the layer above; same workspace
 * size (miq_moe_workspace_bytes). */
int miq_w4a16_moe_routed(const void* hidden, int64_t T, int64_t H, int64_t I, int64_t E, int64_t topk,
                         const uint8_t* gu_q, const void* gu_scale, const void* gu_zero,
                         const uint8_t* dn_q, const void* dn_scale, const void* dn_zero,
                         int sz_dtype, int64_t group, const void* topk_weights, int w_dtype,
                         const void* topk_ids, int idx_dtype, void* workspace, size_t workspace_bytes,
                         void* out, void* stream);
int miq_w8a16_moe_routed(const void* hidden, int64_t T, int64_t H, int64_t I, int64_t E, int64_t topk,
                         const int8_t* gu_q, const void* gu_scale, const int8_t* dn_q, const void* dn_scale,
                         int scale_dtype, const void* topk_weights, int w_dtype,
                         const void* topk_ids, int idx_dtype, void* workspace, size_t workspace_bytes,
                         void* out, void* stream);
int miq_fp8_moe_routed(const void* hidden, int64_t T, int64_t H, int64_t I, int64_t E, int64_t topk,
                       const uint8_t* gu_q, const float* gu_scale, const uint8_t* dn_q, const float* dn_scale,
                       const void* topk_weights, int w_dtype, const void* topk_ids, int idx_dtype,
                       void* workspace, size_t workspace_bytes, void* out, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* MIQ_H_ */
