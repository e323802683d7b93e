// Quantize / dequantize kernels: weights (int8, int4, fp8), fp8 activations and the
// quantize-on-write of 8-bit KV caches. All are bandwidth-bound elementwise + row
// reduction passes; one wavefront or one workgroup per row keeps the row reduction in
// registers (DPP/shuffle) and LDS, and every division is IEEE (correctly rounded), so
// the bytes written equal what the reference's PyTorch formulas produce.
#include "miq_common.h"

namespace miq {
namespace {

constexpr int kRowThreads = 256;

__device__ inline float block_reduce_max(float v, float* red) {
  v = wave_max(v);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  __syncthreads();  // `red` may still be read from a previous reduction
  if (lane == 0) red[wid] = v;
  __syncthreads();
  float r = red[0];
  for (int i = 1; i < (int)(blockDim.x >> 6); ++i) r = fmaxf(r, red[i]);
  return r;
}

// ---------------------------------------------------------------- int8 per-row (int8_wo.py:8-12)
__global__ void __launch_bounds__(kRowThreads)
int8_quantize_kernel(const void* __restrict__ w, int w_dtype, int64_t K, int64_t ldw,
                     int8_t* __restrict__ q, void* __restrict__ scale, int scale_dtype) {
  __shared__ float red[kRowThreads / 64];
  const int64_t row = blockIdx.x;
  const int64_t base = row * ldw;
  float amax = 0.f;
  for (int64_t k = threadIdx.x; k < K; k += blockDim.x)
    amax = fmaxf(amax, fabsf(load_scalar(w, w_dtype, base + k)));
  amax = block_reduce_max(amax, red);
  const float s = fmaxf(amax, 1e-8f) / 127.0f;
  for (int64_t k = threadIdx.x; k < K; k += blockDim.x) {
    float v = __builtin_rintf(load_scalar(w, w_dtype, base + k) / s);
    v = fminf(fmaxf(v, -127.f), 127.f);
    q[row * K + k] = static_cast<int8_t>(v);
  }
  if (threadIdx.x == 0) store_scalar(scale, scale_dtype, row, s);
}

__global__ void int8_dequantize_kernel(const int8_t* __restrict__ q, const void* __restrict__ scale,
                                       int dtype, int64_t rows, int64_t K, void* __restrict__ out) {
  const int64_t n = rows * K;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const float s = load_scalar(scale, dtype, i / K);
    store_scalar(out, dtype, i, static_cast<float>(q[i]) * s);  // one product, one rounding
  }
}

// ---------------------------------------------------------------- int4 group-wise (int4_wo.py:15-42)
// One wavefront per (row, group). zero == nullptr selects the symmetric format used by
// the benchmark configuration: s = max|w| / 7, code = clamp(round(w / s), -8, 7) + 8.
__global__ void __launch_bounds__(64)
int4_quantize_kernel(const void* __restrict__ w, int w_dtype, int64_t K, int64_t ldw, int64_t group,
                     uint8_t* __restrict__ q, void* __restrict__ scale, void* __restrict__ zero,
                     int sz_dtype) {
  const int64_t row = blockIdx.y, g = blockIdx.x, ngroups = K / group;
  const int64_t base = row * ldw + g * group;
  float lo = __builtin_inff(), hi = -__builtin_inff();
  for (int64_t j = threadIdx.x; j < group; j += 64) {
    const float v = load_scalar(w, w_dtype, base + j);
    lo = fminf(lo, v);
    hi = fmaxf(hi, v);
  }
  lo = -wave_max(-lo);
  hi = wave_max(hi);
  const bool sym = zero == nullptr;
  const float s = sym ? fmaxf(fmaxf(hi, -lo) / 7.0f, 1e-8f) : fmaxf((hi - lo) / 15.0f, 1e-8f);
  for (int64_t j = threadIdx.x; j < group / 2; j += 64) {
    const float w0 = load_scalar(w, w_dtype, base + 2 * j);
    const float w1 = load_scalar(w, w_dtype, base + 2 * j + 1);
    float a, b;
    if (sym) {
      a = fminf(fmaxf(__builtin_rintf(w0 / s), -8.f), 7.f) + 8.f;
      b = fminf(fmaxf(__builtin_rintf(w1 / s), -8.f), 7.f) + 8.f;
    } else {
      a = fminf(fmaxf(__builtin_rintf((w0 - lo) / s), 0.f), 15.f);
      b = fminf(fmaxf(__builtin_rintf((w1 - lo) / s), 0.f), 15.f);
    }
    q[row * (K / 2) + (g * group) / 2 + j] =
        static_cast<uint8_t>(static_cast<uint32_t>(a) | (static_cast<uint32_t>(b) << 4));
  }
  if (threadIdx.x == 0) {
    store_scalar(scale, sz_dtype, row * ngroups + g, s);
    if (!sym) store_scalar(zero, sz_dtype, row * ngroups + g, lo);
  }
}

__global__ void int4_dequantize_kernel(const uint8_t* __restrict__ q, const void* __restrict__ scale,
                                       const void* __restrict__ zero, int dtype, int64_t rows,
                                       int64_t K, int64_t group, void* __restrict__ out) {
  const int64_t n = rows * K, ngroups = K / group;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = i / K, k = i - row * K;
    const uint8_t byte = q[row * (K / 2) + k / 2];
    const float u = static_cast<float>((k & 1) ? (byte >> 4) : (byte & 0xf));
    const int64_t gi = row * ngroups + k / group;
    const float s = load_scalar(scale, dtype, gi);
    float v;
    if (zero) {
      v = round_to(round_to(u * s, dtype) + load_scalar(zero, dtype, gi), dtype);
    } else {
      v = round_to((u - 8.f) * s, dtype);
    }
    store_scalar(out, dtype, i, v);
  }
}

// ---------------------------------------------------------------- fp8 rows (fp8.py:32-46)
// e4m3 codes of 8 bf16 values x / s (r = RN(1 / s)): the hardware e4m3 (OCP) conversion
// rounds to nearest even like f32_to_fp8; the inputs are clamped to +-448 first, as the
// reference does
__device__ inline uint2 fp8_encode8(const uint4& p, float s, float r) {
  const uint32_t d[4] = {p.x, p.y, p.z, p.w};
  int o[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    float v[4];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      v[2 * i] = fminf(fmaxf(div_by_recip(bf16_to_f32(d[2 * h + i] & 0xffff), s, r), -448.f), 448.f);
      v[2 * i + 1] = fminf(fmaxf(div_by_recip(bf16_to_f32(d[2 * h + i] >> 16), s, r), -448.f), 448.f);
    }
    o[h] = __builtin_amdgcn_cvt_pk_fp8_f32(v[0], v[1], 0, false);
    o[h] = __builtin_amdgcn_cvt_pk_fp8_f32(v[2], v[3], o[h], true);
  }
  return make_uint2((uint32_t)o[0], (uint32_t)o[1]);
}

__device__ inline float max_abs8(const uint4& p, float amax) {
  const uint32_t d[4] = {p.x, p.y, p.z, p.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    amax = fmaxf(amax, fabsf(bf16_to_f32(d[i] & 0xffff)));
    amax = fmaxf(amax, fabsf(bf16_to_f32(d[i] >> 16)));
  }
  return amax;
}

// bf16 rows of at most 64 * kWaveHeld pieces of 8 (K <= 4096), 16-byte aligned: one
// wavefront per row, the row held in registers between the max and the encode, the max
// reduced across the wavefront (no LDS, no barrier). The codes and the scale are those of
// the workgroup-per-row kernel below (the same maximum and the same expressions).
constexpr int kWaveHeld = 8;
__global__ void __launch_bounds__(kRowThreads)
fp8_quantize_rows_wave_kernel(const uint16_t* __restrict__ x, int64_t K, int64_t ldx, int64_t rows,
                              uint8_t* __restrict__ q, float* __restrict__ scale) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * (kRowThreads / 64) + (threadIdx.x >> 6);
  if (row >= rows) return;  // whole wavefronts
  const uint4* xv = reinterpret_cast<const uint4*>(x + row * ldx);
  const int npc = (int)(K / 8);
  uint4 held[kWaveHeld];
  float amax = 0.f;
#pragma unroll
  for (int j = 0; j < kWaveHeld; ++j) {
    const int c = lane + 64 * j;
    held[j] = c < npc ? xv[c] : make_uint4(0, 0, 0, 0);
  }
#pragma unroll
  for (int j = 0; j < kWaveHeld; ++j) amax = max_abs8(held[j], amax);
  amax = wave_max(amax);
  const float s = fmaxf(amax, 1e-12f) / 448.0f, rs = 1.0f / s;
  uint2* qv = reinterpret_cast<uint2*>(q + row * K);
#pragma unroll
  for (int j = 0; j < kWaveHeld; ++j) {
    const int c = lane + 64 * j;
    if (c < npc) qv[c] = fp8_encode8(held[j], s, rs);
  }
  if (lane == 0) scale[row] = s;
}

__global__ void __launch_bounds__(kRowThreads)
fp8_quantize_rows_kernel(const void* __restrict__ x, int x_dtype, int64_t K, int64_t ldx,
                         uint8_t* __restrict__ q, float* __restrict__ scale) {
  __shared__ float red[kRowThreads / 64];
  const int64_t row = blockIdx.x;
  const int64_t base = row * ldx;
  float amax = 0.f;
  if (x_dtype == MIQ_BF16 && (K % 8) == 0 && (ldx % 8) == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
      (reinterpret_cast<uintptr_t>(q) & 7) == 0) {
    // the row's 8-element pieces: up to kHeld per thread stay in registers between the
    // max pass and the conversion pass (K <= 8192 at 256 threads), later ones are read again
    constexpr int kHeld = 4;
    const uint4* xv = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(x) + base);
    const int64_t npc = K / 8;
    uint4 held[kHeld];
#pragma unroll
    for (int j = 0; j < kHeld; ++j) {
      const int64_t c = threadIdx.x + (int64_t)j * blockDim.x;
      held[j] = c < npc ? xv[c] : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < kHeld; ++j) amax = max_abs8(held[j], amax);
    for (int64_t c = threadIdx.x + (int64_t)kHeld * blockDim.x; c < npc; c += blockDim.x) amax = max_abs8(xv[c], amax);
    amax = block_reduce_max(amax, red);
    const float s = fmaxf(amax, 1e-12f) / 448.0f, rs = 1.0f / s;
    uint2* qv = reinterpret_cast<uint2*>(q + row * K);
#pragma unroll
    for (int j = 0; j < kHeld; ++j) {
      const int64_t c = threadIdx.x + (int64_t)j * blockDim.x;
      if (c < npc) qv[c] = fp8_encode8(held[j], s, rs);
    }
    for (int64_t c = threadIdx.x + (int64_t)kHeld * blockDim.x; c < npc; c += blockDim.x) qv[c] = fp8_encode8(xv[c], s, rs);
    if (threadIdx.x == 0) scale[row] = s;
    return;
  }
  for (int64_t k = threadIdx.x; k < K; k += blockDim.x)
    amax = fmaxf(amax, fabsf(load_scalar(x, x_dtype, base + k)));
  amax = block_reduce_max(amax, red);
  const float s = fmaxf(amax, 1e-12f) / 448.0f;
  for (int64_t k = threadIdx.x; k < K; k += blockDim.x) {
    const float v = fminf(fmaxf(load_scalar(x, x_dtype, base + k) / s, -448.f), 448.f);
    q[row * K + k] = f32_to_fp8(v);
  }
  if (threadIdx.x == 0) scale[row] = s;
}

__global__ void fp8_dequantize_kernel(const uint8_t* __restrict__ q, const float* __restrict__ scale,
                                      int64_t rows, int64_t K, float* __restrict__ out) {
  const int64_t n = rows * K;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    out[i] = fp8_to_f32(q[i]) * scale[i / K];
}

// ---------------------------------------------------------------- KV quantize-on-write
// (kv_cache.py:359-388). One wavefront per (token, head).
__global__ void __launch_bounds__(64)
kv_quant_write_kernel(const void* __restrict__ x, int x_dtype, int64_t heads, int64_t D,
                      int64_t xs_t, int64_t xs_h, const int64_t* __restrict__ slots,
                      uint8_t* __restrict__ cache, int kv_dtype, int64_t cs_t, int64_t cs_h,
                      void* __restrict__ cscale, int scale_dtype, int64_t ss_t, int64_t ss_h) {
  const int64_t t = blockIdx.y, h = blockIdx.x;
  const int64_t xb = t * xs_t + h * xs_h;
  const bool is_int8 = kv_dtype == MIQ_INT8;
  const float qmax = is_int8 ? 127.0f : 448.0f;
  float amax = 0.f;
  for (int64_t d = threadIdx.x; d < D; d += 64) amax = fmaxf(amax, fabsf(load_scalar(x, x_dtype, xb + d)));
  amax = wave_max(amax);
  // the scale is rounded to its storage dtype before it is used, as the reference does
  const float s = round_to(fmaxf(amax / qmax, 1e-8f), scale_dtype);
  const int64_t slot = slots[t];
  uint8_t* dst = cache + slot * cs_t + h * cs_h;
  for (int64_t d = threadIdx.x; d < D; d += 64) {
    const float v = load_scalar(x, x_dtype, xb + d) / s;
    if (is_int8) {
      const float r = fminf(fmaxf(__builtin_rintf(v), -127.f), 127.f);
      dst[d] = static_cast<uint8_t>(static_cast<int8_t>(r));
    } else {
      dst[d] = f32_to_fp8(fminf(fmaxf(v, -448.f), 448.f));
    }
  }
  if (threadIdx.x == 0) store_scalar(cscale, scale_dtype, slot * ss_t + h * ss_h, s);
}

inline bool is_float_dtype(int d) { return d == MIQ_F32 || d == MIQ_BF16 || d == MIQ_F16; }

inline unsigned grid_for(int64_t n) {
  int64_t b = (n + 255) / 256;
  if (b > 65536) b = 65536;
  if (b < 1) b = 1;
  return static_cast<unsigned>(b);
}

}  // namespace
}  // namespace miq

using namespace miq;

extern "C" int miq_int8_quantize(const void* w, int w_dtype, int64_t rows, int64_t K, int64_t ldw,
                                 int8_t* q, void* scale, int scale_dtype, void* stream) {
  MIQ_REQUIRE(is_float_dtype(w_dtype) && is_float_dtype(scale_dtype), "int8_quantize: bad dtype");
  MIQ_REQUIRE(rows >= 0 && K > 0 && ldw >= K, "int8_quantize: bad shape rows=%lld K=%lld ldw=%lld",
              (long long)rows, (long long)K, (long long)ldw);
  if (rows == 0) return MIQ_OK;
  hipLaunchKernelGGL(int8_quantize_kernel, dim3((unsigned)rows), dim3(kRowThreads), 0,
                     (hipStream_t)stream, w, w_dtype, K, ldw, q, scale, scale_dtype);
  return check_launch("int8_quantize");
}

extern "C" int miq_int8_dequantize(const int8_t* q, const void* scale, int scale_dtype, int64_t rows,
                                   int64_t K, void* out, void* stream) {
  MIQ_REQUIRE(is_float_dtype(scale_dtype), "int8_dequantize: bad dtype");
  MIQ_REQUIRE(rows >= 0 && K > 0, "int8_dequantize: bad shape");
  if (rows == 0) return MIQ_OK;
  hipLaunchKernelGGL(int8_dequantize_kernel, dim3(grid_for(rows * K)), dim3(256), 0,
                     (hipStream_t)stream, q, scale, scale_dtype, rows, K, out);
  return check_launch("int8_dequantize");
}

extern "C" int miq_int4_quantize(const void* w, int w_dtype, int64_t rows, int64_t K, int64_t ldw,
                                 int64_t group, uint8_t* q, void* scale, void* zero, int sz_dtype,
                                 void* stream) {
  MIQ_REQUIRE(is_float_dtype(w_dtype) && is_float_dtype(sz_dtype), "int4_quantize: bad dtype");
  MIQ_REQUIRE(group > 0 && group % 2 == 0 && K % group == 0 && ldw >= K,
              "int4_quantize: K=%lld must be a multiple of an even group=%lld", (long long)K,
              (long long)group);
  if (rows == 0) return MIQ_OK;
  MIQ_REQUIRE(rows < 65536 * 1024LL, "int4_quantize: too many rows");
  // rows go on grid.y (limit 65535); larger row counts are split over several launches
  for (int64_t r0 = 0; r0 < rows; r0 += 65535) {
    const int64_t nr = rows - r0 < 65535 ? rows - r0 : 65535;
    const size_t esz = w_dtype == MIQ_F32 ? 4 : 2;
    const size_t ssz = sz_dtype == MIQ_F32 ? 4 : 2;
    hipLaunchKernelGGL(int4_quantize_kernel, dim3((unsigned)(K / group), (unsigned)nr), dim3(64), 0,
                       (hipStream_t)stream, static_cast<const char*>(w) + r0 * ldw * esz, w_dtype,
                       K, ldw, group, q + r0 * (K / 2),
                       static_cast<char*>(scale) + r0 * (K / group) * ssz,
                       zero ? static_cast<char*>(zero) + r0 * (K / group) * ssz : nullptr, sz_dtype);
    int rc = check_launch("int4_quantize");
    if (rc) return rc;
  }
  return MIQ_OK;
}

extern "C" int miq_int4_dequantize(const uint8_t* q, const void* scale, const void* zero, int sz_dtype,
                                   int64_t rows, int64_t K, int64_t group, void* out, void* stream) {
  MIQ_REQUIRE(is_float_dtype(sz_dtype), "int4_dequantize: bad dtype");
  MIQ_REQUIRE(group > 0 && group % 2 == 0 && K % group == 0, "int4_dequantize: bad group");
  if (rows == 0) return MIQ_OK;
  hipLaunchKernelGGL(int4_dequantize_kernel, dim3(grid_for(rows * K)), dim3(256), 0,
                     (hipStream_t)stream, q, scale, zero, sz_dtype, rows, K, group, out);
  return check_launch("int4_dequantize");
}

extern "C" int miq_fp8_quantize_rows(const void* x, int x_dtype, int64_t rows, int64_t K, int64_t ldx,
                                     uint8_t* q, float* scale, void* stream) {
  MIQ_REQUIRE(is_float_dtype(x_dtype), "fp8_quantize_rows: bad dtype");
  MIQ_REQUIRE(K > 0 && ldx >= K && rows >= 0, "fp8_quantize_rows: bad shape");
  if (rows == 0) return MIQ_OK;
  MIQ_REQUIRE(rows <= 0x7fffffff, "fp8_quantize_rows: too many rows");
  if (x_dtype == MIQ_BF16 && K % 8 == 0 && K <= 64 * 8 * kWaveHeld && ldx % 8 == 0 &&
      (reinterpret_cast<uintptr_t>(x) & 15) == 0 && (reinterpret_cast<uintptr_t>(q) & 7) == 0 &&
      !tuning().fp8_quant_rows_wg) {
    const int64_t per = kRowThreads / 64;  // rows per workgroup
    hipLaunchKernelGGL(fp8_quantize_rows_wave_kernel, dim3((unsigned)((rows + per - 1) / per)), dim3(kRowThreads), 0,
                       (hipStream_t)stream, static_cast<const uint16_t*>(x), K, ldx, rows, q, scale);
    return check_launch("fp8_quantize_rows");
  }
  hipLaunchKernelGGL(fp8_quantize_rows_kernel, dim3((unsigned)rows), dim3(kRowThreads), 0,
                     (hipStream_t)stream, x, x_dtype, K, ldx, q, scale);
  return check_launch("fp8_quantize_rows");
}

extern "C" int miq_fp8_dequantize(const uint8_t* q, const float* scale, int64_t rows, int64_t K,
                                  float* out, void* stream) {
  MIQ_REQUIRE(rows >= 0 && K > 0, "fp8_dequantize: bad shape");
  if (rows == 0) return MIQ_OK;
  hipLaunchKernelGGL(fp8_dequantize_kernel, dim3(grid_for(rows * K)), dim3(256), 0,
                     (hipStream_t)stream, q, scale, rows, K, out);
  return check_launch("fp8_dequantize");
}

extern "C" int miq_kv_quant_write(const void* x, int x_dtype, int64_t T, int64_t heads, int64_t D,
                                  int64_t x_stride_t, int64_t x_stride_h, const int64_t* slots,
                                  void* cache, int kv_dtype, int64_t c_stride_t, int64_t c_stride_h,
                                  void* cache_scale, int scale_dtype, int64_t s_stride_t,
                                  int64_t s_stride_h, void* stream) {
  MIQ_REQUIRE(is_float_dtype(x_dtype) && is_float_dtype(scale_dtype), "kv_quant_write: bad dtype");
  MIQ_REQUIRE(kv_dtype == MIQ_INT8 || kv_dtype == MIQ_FP8_E4M3,
              "kv_quant_write: kv_dtype must be int8 or fp8");
  MIQ_REQUIRE(T >= 0 && heads > 0 && D > 0 && heads < 65536 && T < 65536,
              "kv_quant_write: bad shape T=%lld heads=%lld", (long long)T, (long long)heads);
  if (T == 0) return MIQ_OK;
  hipLaunchKernelGGL(kv_quant_write_kernel, dim3((unsigned)heads, (unsigned)T), dim3(64), 0,
                     (hipStream_t)stream, x, x_dtype, heads, D, x_stride_t, x_stride_h, slots,
                     static_cast<uint8_t*>(cache), kv_dtype, c_stride_t, c_stride_h, cache_scale,
                     scale_dtype, s_stride_t, s_stride_h);
  return check_launch("kv_quant_write");
}
