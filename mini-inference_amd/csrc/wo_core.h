// Device-side core shared by the weight-only GEMM (wo_gemm.hip) and the INT4 MoE
// kernels (moe.hip): weight unpacking into MFMA B operands, activation staging into
// LDS, and the per-wavefront K loop over 16 weight rows.
//
// Data layout of one "k-step" (128 k) for the 16 weight rows of a wavefront:
//   lane (r = lane % 16, g = lane / 16) owns weight row n0 + r;
//   int4: one 16-byte load = 32 codes, k = 32 g .. 32 g + 31; MFMA j (0..3) takes the
//         8 codes of word j, k = 32 g + 8 j + (0,4,1,5,2,6,3,7) (see unpack_u4);
//   int8: two 16-byte loads L = 0, 1 = 16 codes each, k = 64 L + 16 g .. + 15; MFMA
//         j = 2 L + h takes bytes 8 h .. 8 h + 7 in natural order.
// The A operand (activations, lane % 16 = row m) is read from LDS at the same k offsets;
// for int4 the activations are stored with the same (0,4,1,5,2,6,3,7) order inside each
// group of 8, so the unpacked codes need no shuffling.
//
// Codes are unpacked to bf16 values 128 + code (exact): int4 by one AND-OR per pair
// (bf16 0x4300 | u == 128 + u), int8 by xor 0x80 and a byte-to-float convert. An extra
// MFMA against ones gives sum x over the same k, and the per-group (int4) or per-row
// (int8) correction removes the 128 offset when scales are applied.
#pragma once
#include "miq_common.h"

namespace miq {
namespace wo {

constexpr int kStepK = 128;
enum { KIND_INT8 = 0, KIND_INT4 = 1 };

__device__ inline bf16x8 as_bf16x8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  i32x4 v = {(int)a, (int)b, (int)c, (int)d};
  return __builtin_bit_cast(bf16x8, v);
}

__device__ inline bf16x8 zero_bf16x8() { return as_bf16x8(0, 0, 0, 0); }

// 8 int4 codes of one 32-bit word -> 8 bf16 values 128 + u in the order
// (k0, k4, k1, k5, k2, k6, k3, k7).
__device__ inline bf16x8 unpack_u4(uint32_t w) {
  const uint32_t m = 0x000f000fu, o = 0x43004300u;
  return as_bf16x8((w & m) | o, ((w >> 4) & m) | o, ((w >> 8) & m) | o, ((w >> 12) & m) | o);
}

// 4 int8 codes -> 2 dwords of bf16 (128 + q), natural order. The integers 0..255 are
// exact in bf16, so keeping the high 16 bits of the float is exact.
__device__ inline void unpack_i8_word(uint32_t w, uint32_t& lo, uint32_t& hi) {
  w ^= 0x80808080u;
  const float f0 = static_cast<float>(w & 0xffu);
  const float f1 = static_cast<float>((w >> 8) & 0xffu);
  const float f2 = static_cast<float>((w >> 16) & 0xffu);
  const float f3 = static_cast<float>(w >> 24);
  lo = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, f1), __builtin_bit_cast(uint32_t, f0), 0x07060302u);
  hi = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, f3), __builtin_bit_cast(uint32_t, f2), 0x07060302u);
}

__device__ inline bf16x8 unpack_i8(uint32_t w0, uint32_t w1) {
  uint32_t a, b, c, d;
  unpack_i8_word(w0, a, b);
  unpack_i8_word(w1, c, d);
  return as_bf16x8(a, b, c, d);
}

// 16-byte streaming load (weights are read once: non-temporal)
__device__ inline uint4 load_nt16(const uint8_t* p) {
  const i32x4 v = __builtin_nontemporal_load(reinterpret_cast<const i32x4*>(p));
  return make_uint4((uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3]);
}

__device__ inline f32x4 mfma(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Permute 8 bf16 (4 dwords, natural order) into (0,4,1,5,2,6,3,7).
__device__ inline uint4 permute_for_u4(uint4 v) {
  uint4 o;
  o.x = __builtin_amdgcn_perm(v.z, v.x, 0x05040100u);  // (x0, x4)
  o.y = __builtin_amdgcn_perm(v.z, v.x, 0x07060302u);  // (x1, x5)
  o.z = __builtin_amdgcn_perm(v.w, v.y, 0x05040100u);  // (x2, x6)
  o.w = __builtin_amdgcn_perm(v.w, v.y, 0x07060302u);  // (x3, x7)
  return o;
}

// A operand (activation row m) for MFMA j of local k-step kl.
template <int KIND>
__device__ inline bf16x8 load_a(const uint16_t* lds, int lds_stride, int m, bool row_ok, int kl, int g, int j) {
  if (!row_ok) return zero_bf16x8();
  int off;
  if (KIND == KIND_INT4) off = kl * kStepK + g * 32 + j * 8;
  else off = kl * kStepK + (j >> 1) * 64 + g * 16 + (j & 1) * 8;
  const uint4 v = *reinterpret_cast<const uint4*>(lds + m * lds_stride + off);
  return as_bf16x8(v.x, v.y, v.z, v.w);
}

// Per-wavefront accumulation state for MT tiles of 16 activation rows.
template <int MT>
struct Acc {
  f32x4 acc[MT];   // scaled result (int4) or raw sum x * (128 + q) (int8)
  f32x4 accg[MT];  // int4: current group's sum x * (128 + u)
  f32x4 xs[MT];    // sum x over the current group (int4) or the whole range (int8)
  __device__ inline void clear() {
    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < MT; ++t) { acc[t] = z; accg[t] = z; xs[t] = z; }
  }
};

struct GroupScales {
  const void* scale;
  const void* zero;  // nullptr: symmetric codes, w = (u - 8) * scale
  int dtype;
  int group_steps;   // k-steps per group
  int64_t row_off;   // index of this lane's row's first group in scale / zero
};

// Accumulate k-steps [kst0, kst0 + nsteps) whose activations sit in LDS at local steps
// 0..nsteps-1 (lds column 0 = k-step kst0). wrow points at this lane's weight row.
// rows_ok(t): whether activation row 16 t + r exists.
template <int KIND, int MT, bool HAS_ZERO>
__device__ inline void run_steps(const uint8_t* wrow, const uint16_t* lds, int lds_stride, int M,
                                 int kst0, int nsteps, int r, int g, const GroupScales& gs,
                                 Acc<MT>& st) {
  const bf16x8 ones = as_bf16x8(0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u);
  constexpr int U = KIND == KIND_INT4 ? 8 : 4;  // k-steps whose weights are in flight together
  constexpr int NL = KIND == KIND_INT4 ? 1 : 2;
  for (int kl0 = 0; kl0 < nsteps; kl0 += U) {
    uint4 wbuf[U][NL];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (kl0 + u < nsteps) {
        const int64_t kst = kst0 + kl0 + u;
        if (KIND == KIND_INT4) {
          wbuf[u][0] = load_nt16(wrow + kst * 64 + g * 16);
        } else {
          wbuf[u][0] = load_nt16(wrow + kst * 128 + g * 16);
          wbuf[u][NL - 1] =
              load_nt16(wrow + kst * 128 + 64 + g * 16);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (kl0 + u >= nsteps) break;
      const int kl = kl0 + u;
      bf16x8 b[4];
      if (KIND == KIND_INT4) {
        b[0] = unpack_u4(wbuf[u][0].x);
        b[1] = unpack_u4(wbuf[u][0].y);
        b[2] = unpack_u4(wbuf[u][0].z);
        b[3] = unpack_u4(wbuf[u][0].w);
      } else {
        b[0] = unpack_i8(wbuf[u][0].x, wbuf[u][0].y);
        b[1] = unpack_i8(wbuf[u][0].z, wbuf[u][0].w);
        b[2] = unpack_i8(wbuf[u][NL - 1].x, wbuf[u][NL - 1].y);
        b[3] = unpack_i8(wbuf[u][NL - 1].z, wbuf[u][NL - 1].w);
      }
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        const int m = t * 16 + r;
        const bool ok = m < M;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const bf16x8 a = load_a<KIND>(lds, lds_stride, m, ok, kl, g, j);
          if (KIND == KIND_INT4) st.accg[t] = mfma(a, b[j], st.accg[t]);
          else st.acc[t] = mfma(a, b[j], st.acc[t]);
          st.xs[t] = mfma(a, ones, st.xs[t]);
        }
      }
      if (KIND == KIND_INT4) {
        const int kst = kst0 + kl;
        if ((kst + 1) % gs.group_steps == 0) {  // end of a quantization group
          const int64_t gi = gs.row_off + kst / gs.group_steps;
          const float sc = load_scalar(gs.scale, gs.dtype, gi);
          const float cz = HAS_ZERO ? load_scalar(gs.zero, gs.dtype, gi) - 128.f * sc : -136.f * sc;
          const f32x4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int t = 0; t < MT; ++t) {
#pragma unroll
            for (int v = 0; v < 4; ++v) st.acc[t][v] += sc * st.accg[t][v] + cz * st.xs[t][v];
            st.accg[t] = z;
            st.xs[t] = z;
          }
        }
      }
    }
  }
}

// int8: remove the +128 offset once the whole K range is accumulated
template <int MT>
__device__ inline void finish_int8(Acc<MT>& st) {
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int v = 0; v < 4; ++v) st.acc[t][v] -= 128.f * st.xs[t][v];
}

}  // namespace wo
}  // namespace miq
