// Shared device/host helpers for libmiq (gfx950 only).
//
// Numeric conventions follow what PyTorch does on the CPU for the same formulas:
//   * bf16 values are stored as raw uint16 and widened by a 16-bit shift (exact);
//   * float -> bf16 is round-to-nearest-even (torch's c10::BFloat16 constructor);
//   * float -> e4m3fn is round-to-nearest-even with subnormals (torch's
//     Float8_e4m3fn constructor) for inputs already clamped to +-448.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/miq.h"

namespace miq {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));

__host__ __device__ inline float bf16_to_f32(uint16_t h) {
  union { uint32_t u; float f; } v;
  v.u = static_cast<uint32_t>(h) << 16;
  return v.f;
}

// x / s rounded to nearest, given r = RN(1 / s): q = RN(x r) is within an ulp of x / s,
// and then RN(q + RN(x - q s) r) is the correctly rounded quotient (Markstein's theorem;
// both corrections are fused multiply-adds, so this is three operations instead of the
// division sequence). Valid while x / s and the residual stay in the normal range, which
// holds for activation quantization (|x / s| <= 448 up to rounding; results below the
// normal range become e4m3 zero either way). s > 0, so the quotient carries the sign of x;
// copying it back keeps -0 / s = -0 (the last add would give +0 there).
__device__ inline float div_by_recip(float x, float s, float r) {
  const float q = x * r;
  return __builtin_copysignf(__builtin_fmaf(__builtin_fmaf(-q, s, x), r, q), x);
}

__host__ __device__ inline uint16_t f32_to_bf16(float f) {
  union { uint32_t u; float f; } v;
  v.f = f;
  uint32_t u = v.u;
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return 0x7fc0;  // NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__host__ __device__ inline float f16_to_f32(uint16_t h) {
  return static_cast<float>(*reinterpret_cast<const _Float16*>(&h));
}

__host__ __device__ inline uint16_t f32_to_f16(float f) {
  _Float16 h = static_cast<_Float16>(f);
  return *reinterpret_cast<uint16_t*>(&h);
}

// e4m3fn decode: 1 sign, 4 exponent (bias 7), 3 mantissa bits; 0x7f/0xff are NaN.
__host__ __device__ inline float fp8_to_f32(uint8_t b) {
  const uint32_t s = b & 0x80u, e = (b >> 3) & 0xfu, m = b & 0x7u;
  float mag;
  if (e == 0) {
    mag = static_cast<float>(m) * 0.001953125f;  // m * 2^-9
  } else if (e == 15 && m == 7) {
    mag = __builtin_nanf("");
  } else {
    union { uint32_t u; float f; } v;
    v.u = ((e + 120u) << 23) | (m << 20);  // (1 + m/8) * 2^(e-7)
    mag = v.f;
  }
  return s ? -mag : mag;
}

// e4m3fn encode, round-to-nearest-even, for |x| <= 448 (callers clamp first, as the
// reference formulas do). Subnormals (|x| < 2^-6) are multiples of 2^-9.
__host__ __device__ inline uint8_t f32_to_fp8(float x) {
  union { uint32_t u; float f; } v;
  v.f = x;
  const uint32_t sign = (v.u >> 24) & 0x80u;
  const uint32_t a = v.u & 0x7fffffffu;
  if (a > 0x7f800000u) return static_cast<uint8_t>(sign | 0x7f);  // NaN
  if (a < 0x3c800000u) {  // below 2^-6: subnormal grid of 2^-9
    v.u = a;
    const float q = __builtin_rintf(v.f * 512.0f);  // exact scaling, RNE
    return static_cast<uint8_t>(sign | static_cast<uint32_t>(q));  // q == 8 encodes 2^-6
  }
  // normal: keep 3 mantissa bits with RNE on the 20 dropped bits
  const uint32_t r = a + 0x7ffffu + ((a >> 20) & 1u);
  const uint32_t e = (r >> 23) - 120u;  // rebias 127 -> 7
  const uint32_t m = (r >> 20) & 7u;
  uint32_t code = (e << 3) | m;
  if (code > 0x7eu) code = 0x7eu;  // saturate at 448 (inputs are clamped, kept for safety)
  return static_cast<uint8_t>(sign | code);
}

// Raw bits of element i of a bf16 / f16 / f32 array (SD = the MIQ_* dtype). The value is
// decoded by sd_to_f32 where it is used, so a pending load never forces a wait where it
// is issued (a decode inside a dtype branch would make the compiler wait for all
// outstanding loads right there).
template <int SD>
__device__ inline uint32_t load_sd_raw(const void* p, int64_t i) {
  if constexpr (SD == MIQ_F32) return static_cast<const uint32_t*>(p)[i];
  else return static_cast<const uint16_t*>(p)[i];
}

template <int SD>
__device__ inline float sd_to_f32(uint32_t raw) {
  if constexpr (SD == MIQ_F32) return __builtin_bit_cast(float, raw);
  else if constexpr (SD == MIQ_BF16) return __builtin_bit_cast(float, raw << 16);
  else return f16_to_f32(static_cast<uint16_t>(raw));
}

__device__ inline float load_scalar(const void* p, int dtype, int64_t i) {
  switch (dtype) {
    case MIQ_BF16: return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
    case MIQ_F16: return f16_to_f32(static_cast<const uint16_t*>(p)[i]);
    default: return static_cast<const float*>(p)[i];
  }
}

// Round a float to the storage precision of `dtype` and back.
__device__ inline float round_to(float f, int dtype) {
  switch (dtype) {
    case MIQ_BF16: return bf16_to_f32(f32_to_bf16(f));
    case MIQ_F16: return f16_to_f32(f32_to_f16(f));
    default: return f;
  }
}

__device__ inline void store_scalar(void* p, int dtype, int64_t i, float f) {
  switch (dtype) {
    case MIQ_BF16: static_cast<uint16_t*>(p)[i] = f32_to_bf16(f); break;
    case MIQ_F16: static_cast<uint16_t*>(p)[i] = f32_to_f16(f); break;
    default: static_cast<float*>(p)[i] = f; break;
  }
}

// v gathered from lane addr / 4 (ds_bpermute: the LDS crossbar, no LDS memory)
__device__ inline uint4 bpermute16(int addr, const uint4& v) {
  uint4 o;
  o.x = (uint32_t)__builtin_amdgcn_ds_bpermute(addr, (int)v.x);
  o.y = (uint32_t)__builtin_amdgcn_ds_bpermute(addr, (int)v.y);
  o.z = (uint32_t)__builtin_amdgcn_ds_bpermute(addr, (int)v.z);
  o.w = (uint32_t)__builtin_amdgcn_ds_bpermute(addr, (int)v.w);
  return o;
}

// Two loads of 8 rows x 128 bytes in address order (lane 32 c2 + 4 rr + cl: row 8h + rr of
// load h, bytes 64 c2 + 16 cl) to the MFMA layout: f0 = the first 64-byte half (c2 = 0), f1 = the
// second, lane (g, r) holding row r, chunk g. The 32-lane swap makes register j hold half
// c2 = j with lane bit 5 = h; one gather per dword then rotates the lane bits.
__device__ inline void lanes_to_mfma(int addr, const uint4& l0, const uint4& l1, uint4& f0, uint4& f1) {
  uint4 a, b;
  const uint32_t* p0 = &l0.x;
  const uint32_t* p1 = &l1.x;
  uint32_t* pa = &a.x;
  uint32_t* pb = &b.x;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const auto s = __builtin_amdgcn_permlane32_swap(p0[i], p1[i], false, false);
    pa[i] = s[0];
    pb[i] = s[1];
  }
  f0 = bpermute16(addr, a);
  f1 = bpermute16(addr, b);
}

__device__ inline float wave_max(float v) {
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

__device__ inline float wave_sum(float v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

}  // namespace miq

// ----------------------------------------------------------------- host-side error plumbing
namespace miq {
void set_error(const char* fmt, ...);
int check_launch(const char* what);

// Kernel-selection switches for tests and tuning, read from MIQ_* environment variables
// once at load time (miq_tuning_reload re-reads them); the defaults are the measured best.
struct Tuning {
  bool wo_stream;             // MIQ_WO_STREAM: weight-only GEMMs take the streamed kernel
  int wo_rows;                // MIQ_WO_ROWS: rows per tile of the tile kernel (0: default)
  int wo_tile_min_w;          // MIQ_WO_TILE_MIN_W: fewest wavefronts per tile workgroup (0: planned)
  int wo_pair_min_m;          // MIQ_WO_PAIR_MIN_M: the tile kernel's two-half int4 plan from
                              // this M up to 16 (0: default range, -1: never)
  int wo_int8_tile2_min_m;    // MIQ_WO_INT8_TILE2_MIN_M: int8 tile kernel with two row tiles per
                              // workgroup from this M up to 16 (0: default range, -1: never)
  bool wo_msplit_set;         // MIQ_WO_MSPLIT="NR,S": M-split plan of the streamed kernel
  int wo_msplit_nr, wo_msplit_s;
  bool wo_plan_set;           // MIQ_WO_PLAN="NR,S": plan of the streamed kernel
  int wo_plan_nr, wo_plan_s;
  int wo_panel;               // MIQ_WO_PANEL: 0 off, 1 forced where it applies, -1 default
  int wo_panel_s;             // MIQ_WO_PANEL_S: K splits of the panel kernel (0: planned)
  int wo_panel_mt;            // MIQ_WO_PANEL_MT: activation tiles per panel workgroup (1, 2, 4)
  int wo_gemv_max_m;          // MIQ_WO_GEMV_MAX_M: largest M for the GEMV kernel (0: off, -1: default 1)
  int wo_gemv_waves;          // MIQ_WO_GEMV_WAVES: wavefronts per GEMV workgroup (0: planned)
  int wo_prefill_min_m;       // MIQ_WO_PREFILL_MIN_M: smallest M for the prefill kernel (65)
  int wo_prefill_s;           // MIQ_WO_PREFILL_S: K splits of the prefill kernel (0: planned)
  int wo_wide_mt;             // MIQ_WO_WIDE_MT: 32-row activation tiles per wavefront of the wide kernel
                              // (1..3 forced, 0 off, -1 planned)
  int wo_wide_min_m;          // MIQ_WO_WIDE_MIN_M: smallest M for the wide kernel (65)
  int wo_wide_s;              // MIQ_WO_WIDE_S: K splits of the wide kernel (0: planned)
  bool fp8_old;               // MIQ_FP8_OLD: the previous FP8 GEMM kernel family
  bool fp8_four_waves;        // MIQ_FP8_WAVES=4
  bool fp8_quant_rows_wg;     // MIQ_FP8_QUANT_ROWS_WG: one workgroup per row in fp8_quantize_rows
  bool moe_tiled;             // MIQ_MOE_TILED: the tiled expert kernels
  bool moe_four_waves;        // MIQ_MOE_WAVES=4: four-wavefront streaming expert workgroups
  bool moe_no_lds_scales;     // MIQ_MOE_LDS_SCALES=0: per-k-step scale loads instead of LDS
  bool moe_align_scan;        // MIQ_MOE_ALIGN_SCAN: the one-wavefront-per-expert align
  bool moe_align_launch;      // MIQ_MOE_ALIGN_LAUNCH: routed MoE entry points run moe_align
};
const Tuning& tuning();

// The current device's error word (bits MIQ_DEVERR_*): kernels that detect a condition
// they cannot report through a return code set a bit here; miq_device_errors() reads and
// clears it. The address comes from hipGetSymbolAddress once per device.
unsigned* device_error_word();

// Raises a kernel's dynamic LDS limit to what gfx950's 160 KiB leaves beside its static
// LDS; call once per kernel (a rejected request would otherwise linger as the error the
// next launch check reports, so any error of these calls is consumed here).
inline void allow_max_dynamic_lds(const void* kernel) {
  hipFuncAttributes a{};
  if (hipFuncGetAttributes(&a, kernel) == hipSuccess)
    (void)hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024 - (int)a.sharedSizeBytes);
  (void)hipGetLastError();
}
}  // namespace miq

// Sets `bits` in the device error word (a vector atomic; never a scalar-cache store).
__device__ inline void raise_device_error(unsigned* word, unsigned bits) {
  if (word) __hip_atomic_fetch_or(word, bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

#define MIQ_REQUIRE(cond, ...)                 \
  do {                                         \
    if (!(cond)) {                             \
      ::miq::set_error(__VA_ARGS__);           \
      return MIQ_ERR_INVALID;                  \
    }                                          \
  } while (0)
