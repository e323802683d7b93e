// Decode-shaped (1 <= M <= 16) weight-only GEMM for gfx950: the streaming kernel behind
// miq_w8a16_gemm / miq_w4a16_gemm for one tile of activation rows.
//
// A workgroup owns 16 weight rows and a K range (one of S splits along grid.y); its WK
// wavefronts take contiguous k slices of at most kMaxSteps k-steps (128 k each), so a
// wavefront's whole slice is one batch of weight loads. Every global load is issued
// unconditionally (out-of-range indices are clamped to a valid element and the value is
// ignored), which keeps the number of loads in flight static: the compiler can then wait
// for exactly the data it consumes instead of for everything. The order is
//   1. activation pieces of the workgroup's K range (to be staged in LDS),
//   2. the wavefront's weight slice (16-byte non-temporal loads) and int4 group scales,
//   3. LDS writes of the activations (waits only for step 1), one barrier,
//   4. unpack + MFMA per k-step as the weights arrive, group scale application,
//   5. LDS sum of the WK wavefronts' accumulators, bf16 store (or split-K partials).
// so a workgroup costs one memory round trip. Rows m >= M of the A operand re-read row
// M - 1: MFMA rows are independent and those output rows are never stored.
//
// The sum of the activations needed to remove the +128 code offset comes from an MFMA
// against a B operand of ones on the same A fragments.
#include <stdio.h>
#include <stdlib.h>

#include "wo_core.h"

namespace miq {
namespace {

using namespace wo;

constexpr int kDecWaves = 8;       // at most 8 wavefronts per workgroup
constexpr int kXPieces = 4;        // activation pieces (16 bytes) per thread per round

struct DecParams {
  const uint16_t* x;
  int64_t ldx;
  const uint8_t* w;
  int64_t ldw;  // bytes per weight row
  const void* scale;
  const void* zero;
  int group_steps;
  int64_t ngroups;
  uint16_t* y;
  int64_t ldy;
  int M, N;
  int S, units, unit_steps;
  int range_steps;  // k-steps staged per workgroup (max over splits)
  float* partial;
  int* counters;
};

template <int KIND>
struct DecSteps {
  static constexpr int kMax = KIND == KIND_INT4 ? 16 : 8;  // k-steps per wavefront batch
};

template <int KIND, bool HZ, int SD>
__global__ void __launch_bounds__(kDecWaves * 64)
wo_decode_kernel(DecParams p) {
  extern __shared__ __align__(16) uint16_t lds[];
  constexpr int U = DecSteps<KIND>::kMax;
  constexpr int NL = KIND == KIND_INT4 ? 1 : 2;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int WK = blockDim.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int n = n0 + r;
  const uint8_t* wrow = p.w + (int64_t)n * p.ldw;

  // K range of this split and this wavefront's slice, in whole units
  const int s = blockIdx.y;
  const int u0 = (int)((int64_t)p.units * s / p.S), u1 = (int)((int64_t)p.units * (s + 1) / p.S);
  const int st0 = u0 * p.unit_steps, st1 = u1 * p.unit_steps;
  const int a = (u0 + (int)((int64_t)(u1 - u0) * wv / WK)) * p.unit_steps;
  const int b = (u0 + (int)((int64_t)(u1 - u0) * (wv + 1) / WK)) * p.unit_steps;

  // 1. activation pieces of [st0, st1) for rows < M (first round)
  const int lds_stride = p.range_steps * kStepK + 8;
  const int xcols = (st1 - st0) * (kStepK / 8);
  const int npieces = p.M * xcols;
  const uint4* xsrc = reinterpret_cast<const uint4*>(p.x + (int64_t)st0 * kStepK);
  const int xld = (int)(p.ldx / 8);
  uint4 xv[kXPieces];
#ifndef ABL_NOSTAGE
#pragma unroll
  for (int j = 0; j < kXPieces; ++j) {
    const int i = min(tid + j * (int)blockDim.x, npieces - 1);
    const int m = i / xcols, c = i - m * xcols;
    xv[j] = xsrc[(int64_t)m * xld + c];
  }
#endif

  f32x4 acc = {0.f, 0.f, 0.f, 0.f}, accg = acc, xs = acc;
  const f32x4 z4 = acc;
  const bf16x8 ones = as_bf16x8(0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u);

  for (int k0 = a; k0 < b || k0 == a; k0 += U) {
    // 2. weights and group scales of this batch (all issued, indices clamped)
    const int kend = b;
    uint4 wb[U][NL];
    uint32_t sraw[U], zraw[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kst = max(min(k0 + u, kend - 1), 0);
#pragma unroll
      for (int L = 0; L < NL; ++L) wb[u][L] = load_nt16(wrow + w_off<KIND>(kst, g, L));
#ifdef ABL_NOSCALE
      if (false) {
#else
      if (KIND == KIND_INT4) {
#endif
        const int64_t gi = (int64_t)n * p.ngroups + kst / p.group_steps;
        sraw[u] = load_sd_raw<SD>(p.scale, gi);
        zraw[u] = HZ ? load_sd_raw<SD>(p.zero, gi) : 0u;
      }
    }
#ifdef ABL_NOSCALE
#pragma unroll
    for (int u = 0; u < U; ++u) { sraw[u] = 0x3f80u; zraw[u] = 0; }
#endif
#ifdef ABL_NOSTAGE
    if (k0 == a) { __syncthreads(); if (a >= b) break; }
    if (false) {
#else
    if (k0 == a) {
#endif
      // 3. stage the activations (waits only for the pieces issued first)
#pragma unroll
      for (int j = 0; j < kXPieces; ++j) {
        const int i = tid + j * (int)blockDim.x;
        if (i < npieces) {
          const int m = i / xcols, c = i - m * xcols;
          *reinterpret_cast<uint4*>(lds + m * lds_stride + c * 8) = KIND == KIND_INT4 ? permute_for_u4(xv[j]) : xv[j];
        }
      }
      for (int first = kXPieces * blockDim.x; first < npieces; first += kXPieces * blockDim.x) {
        uint4 mv[kXPieces];
#pragma unroll
        for (int j = 0; j < kXPieces; ++j) {
          const int i = min(first + tid + j * (int)blockDim.x, npieces - 1);
          const int m = i / xcols, c = i - m * xcols;
          mv[j] = xsrc[(int64_t)m * xld + c];
        }
#pragma unroll
        for (int j = 0; j < kXPieces; ++j) {
          const int i = first + tid + j * (int)blockDim.x;
          if (i < npieces) {
            const int m = i / xcols, c = i - m * xcols;
            *reinterpret_cast<uint4*>(lds + m * lds_stride + c * 8) = KIND == KIND_INT4 ? permute_for_u4(mv[j]) : mv[j];
          }
        }
      }
      __syncthreads();
      if (a >= b) break;
    }
    // 4. multiply
#ifdef ABL_NOCOMPUTE
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (k0 + u < kend) acc[0] += __builtin_bit_cast(float, wb[u][0].x ^ wb[u][0].w ^ sraw[u]);
    continue;
#endif
    const uint16_t* arow = lds + min(r, p.M - 1) * lds_stride;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kst = k0 + u;
      if (kst < kend) {  // a guard, not a break: the loop must unroll fully (register arrays)
      const int kl = kst - st0;
      bf16x8 av[4], bv[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint4 v = *reinterpret_cast<const uint4*>(arow + a_off<KIND>(kl, g, j));
        av[j] = as_bf16x8(v.x, v.y, v.z, v.w);
      }
      unpack_b<KIND>(wb[u], bv);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        xs = mfma(av[j], ones, xs);
        if (KIND == KIND_INT4) accg = mfma(av[j], bv[j], accg);
        else acc = mfma(av[j], bv[j], acc);
      }
      if (KIND == KIND_INT4 && (kst + 1) % p.group_steps == 0) {
        const float sc = sd_to_f32<SD>(sraw[u]);
        const float cz = HZ ? sd_to_f32<SD>(zraw[u]) - 128.f * sc : -136.f * sc;
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[v] += sc * accg[v] + cz * xs[v];
        accg = z4;
        xs = z4;
      }
      }
    }
  }
  if (KIND == KIND_INT8) {
#pragma unroll
    for (int v = 0; v < 4; ++v) acc[v] -= 128.f * xs[v];
  }

  // 5. add the wavefronts' accumulators (reusing the activation LDS)
#ifdef ABL_NORED
  if (wv == 0 && g == 0) p.y[n] = f32_to_bf16(acc[0]);
  return;
#endif
  __syncthreads();
  float* red = reinterpret_cast<float*>(lds);
#pragma unroll
  for (int v = 0; v < 4; ++v) red[(wv * 64 + lane) * 4 + v] = acc[v];
  __syncthreads();
  const bool split = p.S > 1;
  for (int e = tid; e < 256; e += blockDim.x) {
    const int v = e & 3, ln = e >> 2;
    const int m = (ln >> 4) * 4 + v, nn = n0 + (ln & 15);
    float o = 0.f;
    for (int w = 0; w < WK; ++w) o += red[(w * 64 + ln) * 4 + v];
    if (m < p.M) {
      if (split) {
        __hip_atomic_store(p.partial + ((int64_t)s * p.M + m) * p.N + nn, o, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      } else {
        if (KIND == KIND_INT8)
          o = bf16_to_f32(f32_to_bf16(o)) * bf16_to_f32(f32_to_bf16(sd_to_f32<SD>(load_sd_raw<SD>(p.scale, nn))));
        p.y[(int64_t)m * p.ldy + nn] = f32_to_bf16(o);
      }
    }
  }
  if (!split) return;
  __builtin_amdgcn_s_waitcnt(0);  // this thread's partial stores have completed
  __syncthreads();
  __shared__ int s_last;
  if (tid == 0)
    s_last = __hip_atomic_fetch_add(p.counters + blockIdx.x, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == p.S - 1;
  __syncthreads();
  if (!s_last) return;
  for (int i = tid; i < p.M * 16; i += blockDim.x) {
    const int m = i >> 4, nn = n0 + (i & 15);
    float o = 0.f;
    for (int ss = 0; ss < p.S; ++ss)
      o += __hip_atomic_load(p.partial + ((int64_t)ss * p.M + m) * p.N + nn, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (KIND == KIND_INT8)
      o = bf16_to_f32(f32_to_bf16(o)) * bf16_to_f32(f32_to_bf16(sd_to_f32<SD>(load_sd_raw<SD>(p.scale, nn))));
    p.y[(int64_t)m * p.ldy + nn] = f32_to_bf16(o);
  }
  if (tid == 0) __hip_atomic_store(p.counters + blockIdx.x, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int KIND, bool HZ, int SD>
void launch_dec(const DecParams& p, dim3 grid, int WK, size_t lds, hipStream_t st) {
  static bool attr = false;
  if (!attr) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&wo_decode_kernel<KIND, HZ, SD>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, 152 * 1024);
    attr = true;
  }
  hipLaunchKernelGGL((wo_decode_kernel<KIND, HZ, SD>), grid, dim3(64 * WK), lds, st, p);
}

}  // namespace

// Plan and launch for 1 <= M <= 16 (called by the miq_w*a16_gemm entry points).
// Returns -1 when the shape needs the general kernel.
int wo_decode_launch(int kind, const uint16_t* x, int64_t ldx, const uint8_t* w, int64_t ldw, const void* scale,
                     const void* zero, int sd, int group_steps, int64_t ngroups, uint16_t* y, int64_t ldy, int M, int N,
                     int K, void* workspace, size_t ws_bytes, size_t counter_bytes, hipStream_t st) {
  if (M < 1 || M > 16) return -1;
  const int steps = K / kStepK;
  const int unit_steps = kind == KIND_INT4 ? group_steps : 1;
  const int units = steps / unit_steps;
  const int tiles = N / 16;
  const int umax = kind == KIND_INT4 ? DecSteps<KIND_INT4>::kMax : DecSteps<KIND_INT8>::kMax;
  // wavefronts per workgroup and K splits: every wavefront's slice fits one batch, and
  // about 2 workgroups per CU when the row tiles allow it
  int WK = 4, S = 1;
  const char* env = getenv("MIQ_DEC_PLAN");
  int ew = 0, es = 0;
  if (env && sscanf(env, "%d,%d", &ew, &es) == 2 && ew >= 1 && ew <= kDecWaves && es >= 1) {
    WK = ew;
    S = es;
  } else {
    while ((int64_t)WK * S * umax < steps) {
      if (WK < kDecWaves) WK *= 2;
      else ++S;
    }
    while (tiles * S < 512 && S * WK * 2 <= units && WK > 1 && (int64_t)tiles * S * 2 <= 4096) {
      // more splits when the row tiles alone leave CUs idle
      S *= 2;
      if ((int64_t)(WK / 2) * S * umax >= steps) WK /= 2;
    }
  }
  if (S > units) S = units;
  if (tiles > 4096) S = 1;
  // the activation range must fit in LDS
  while ((size_t)M * (((units + S - 1) / S) * unit_steps * kStepK + 8) * 2 > 150 * 1024 && S < units && tiles <= 4096)
    S *= 2;
  if (S > units) S = units;
  const int range_units = (units + S - 1) / S;
  const int range_steps = range_units * unit_steps;
  const size_t lds_x = (size_t)M * (range_steps * kStepK + 8) * 2;
  const size_t lds_red = (size_t)WK * 64 * 4 * 4;
  const size_t lds = lds_x > lds_red ? lds_x : lds_red;
  if (lds > 152 * 1024) return -1;
  const size_t need = counter_bytes + (S > 1 ? (size_t)S * M * N * 4 : 0);
  if (S > 1 && (workspace == nullptr || ws_bytes < need)) return -1;
  DecParams p{};
  p.x = x;
  p.ldx = ldx;
  p.w = w;
  p.ldw = ldw;
  p.scale = scale;
  p.zero = zero;
  p.group_steps = group_steps;
  p.ngroups = ngroups;
  p.y = y;
  p.ldy = ldy;
  p.M = M;
  p.N = N;
  p.S = S;
  p.units = units;
  p.unit_steps = unit_steps;
  p.range_steps = range_steps;
  p.counters = static_cast<int*>(workspace);
  p.partial = workspace ? reinterpret_cast<float*>(static_cast<char*>(workspace) + counter_bytes) : nullptr;
  const dim3 grid((unsigned)tiles, (unsigned)S);
#define MIQ_DEC(K_, HZ_, SD_) launch_dec<K_, HZ_, SD_>(p, grid, WK, lds, st)
  if (kind == KIND_INT8) {
    if (sd == MIQ_BF16) MIQ_DEC(KIND_INT8, false, MIQ_BF16);
    else if (sd == MIQ_F16) MIQ_DEC(KIND_INT8, false, MIQ_F16);
    else MIQ_DEC(KIND_INT8, false, MIQ_F32);
  } else if (zero) {
    if (sd == MIQ_BF16) MIQ_DEC(KIND_INT4, true, MIQ_BF16);
    else if (sd == MIQ_F16) MIQ_DEC(KIND_INT4, true, MIQ_F16);
    else MIQ_DEC(KIND_INT4, true, MIQ_F32);
  } else {
    if (sd == MIQ_BF16) MIQ_DEC(KIND_INT4, false, MIQ_BF16);
    else if (sd == MIQ_F16) MIQ_DEC(KIND_INT4, false, MIQ_F16);
    else MIQ_DEC(KIND_INT4, false, MIQ_F32);
  }
#undef MIQ_DEC
  return check_launch(kind == KIND_INT8 ? "w8a16_gemm" : "w4a16_gemm");
}

}  // namespace miq
