// Device-side core shared by the weight-only GEMM (wo_gemm.hip) and the INT4 MoE
// kernels (moe.hip): weight unpacking into MFMA B operands and the per-wavefront
// accumulation over k-steps.
//
// Data layout of one "k-step" (128 k) for a tile of 16 weight rows:
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
// (bf16 0x4300 | u == 128 + u), int8 by xor 0x80 and a byte-to-float convert. The sums
// of the activations over each group (int4) or over the whole range (int8), computed
// once per workgroup from the staged activations, remove the 128 offset when the
// scales are applied.
#pragma once
#include <type_traits>



#include "miq_common.h"

namespace miq {
namespace wo {

constexpr int kStepK = 128;
enum { KIND_INT8 = 0, KIND_INT4 = 1 };

// k-steps per weight batch (UB KiB of int4 or int8 weights per wavefront)
template <int KIND, int NT, int UB>
__host__ __device__ constexpr int batch_steps() {
  return KIND == KIND_INT4 ? UB / NT : UB / (2 * NT);
}

__device__ inline bf16x8 as_bf16x8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  i32x4 v = {(int)a, (int)b, (int)c, (int)d};
  return __builtin_bit_cast(bf16x8, v);
}

__device__ inline bf16x8 zero_bf16x8() { return as_bf16x8(0, 0, 0, 0); }

// 8 int4 codes of one 32-bit word -> 8 bf16 values 128 + u in the order
// (k0, k4, k1, k5, k2, k6, k3, k7).
// The mask and the bias are passed through empty asm statements so that they sit in
// registers: (x & m) | o is then one v_and_or_b32 (a three-operand VALU instruction cannot
// carry literal constants on gfx9), seven VALU operations per word instead of eleven.
__device__ inline bf16x8 unpack_u4(uint32_t w) {
  uint32_t m, o;
  asm("" : "=s"(m) : "0"(0x000f000fu));
  asm("" : "=v"(o) : "0"(0x43004300u));
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

// Byte offset, inside a 16-row weight tile's row, of k-step `kst`, for load L.
template <int KIND>
__device__ inline int64_t w_off(int64_t kst, int g, int L) {
  return KIND == KIND_INT4 ? kst * 64 + g * 16 : kst * 128 + L * 64 + g * 16;
}

// Element offset inside an activation row (LDS) of MFMA j of local k-step kl.
template <int KIND>
__device__ inline int a_off(int kl, int g, int j) {
  return KIND == KIND_INT4 ? kl * kStepK + g * 32 + j * 8 : kl * kStepK + (j >> 1) * 64 + g * 16 + (j & 1) * 8;
}

template <int KIND>
__device__ inline void unpack_b(const uint4* w, bf16x8 b[4]) {
  if (KIND == KIND_INT4) {
    b[0] = unpack_u4(w[0].x);
    b[1] = unpack_u4(w[0].y);
    b[2] = unpack_u4(w[0].z);
    b[3] = unpack_u4(w[0].w);
  } else {
    b[0] = unpack_i8(w[0].x, w[0].y);
    b[1] = unpack_i8(w[0].z, w[0].w);
    b[2] = unpack_i8(w[1].x, w[1].y);
    b[3] = unpack_i8(w[1].z, w[1].w);
  }
}


// Sum of the 8 bf16 values of a 16-byte piece: four dot products with (1, 1) (exact
// products, fp32 sums)
__device__ inline float sum8_bf16(uint4 v) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  const bf16x2 one = {static_cast<__bf16>(1.0f), static_cast<__bf16>(1.0f)};
  const float a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, v.x), one, 0.f, false);
  const float b = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, v.z), one, 0.f, false);
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, v.w), one,
                                         __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, v.y), one, a, false),
                                         false) + b;
}

// The aligned 32-bit word holding element i of a bf16 / f16 / f32 array (a 16-bit load
// would be widened right where it is issued, which makes the compiler wait for it), and
// the element's value from that word.
template <int SD>
__device__ inline uint32_t load_sd_word(const void* p, int64_t i) {
  if constexpr (SD == MIQ_F32) return static_cast<const uint32_t*>(p)[i];
  else return static_cast<const uint32_t*>(p)[i >> 1];
}

template <int SD>
__device__ inline float word_to_f32(uint32_t w, int64_t i) {
  if constexpr (SD == MIQ_F32) return __builtin_bit_cast(float, w);
  else return sd_to_f32<SD>((i & 1) ? (w >> 16) : (w & 0xffffu));
}

// int4 group scales / zeros of the workgroup's rows, staged in LDS as raw bits:
// sc[row * stride + (group - g0)], row = 16 t + r (NT tiles), groups g0 .. g0 + stride - 1.
template <int SD>
struct GroupQ {
  typedef typename std::conditional<SD == MIQ_F32, uint32_t, uint16_t>::type raw_t;
  const raw_t* sc;
  const raw_t* zr;   // nullptr: symmetric codes, w = (u - 8) * scale
  int stride;        // groups per staged row
  int g0;            // first staged group
  int group_steps;   // k-steps per quantization group
  const float* xsum; // int4: sum of x over each staged group, [group - g0][16 * MT rows]
  int xrows;         // 16 * MT
};

// Stage the scale (and zero) rows [row0, row0 + nrows) x groups [g0, g0 + ng) of a
// [rows, ngroups] array into LDS (raw bits); all threads of the workgroup take part.
template <int SD>
__device__ inline void stage_groups(const void* src, int64_t ngroups, int64_t row0, int nrows, int g0, int ng,
                                    typename GroupQ<SD>::raw_t* dst) {
  typedef typename GroupQ<SD>::raw_t raw_t;
  const raw_t* s = static_cast<const raw_t*>(src);
  for (int i = threadIdx.x; i < nrows * ng; i += blockDim.x) {
    const int rr = i / ng, c = i - rr * ng;
    dst[i] = s[(row0 + rr) * ngroups + g0 + c];
  }
}

// Two-phase staging of a [rows, cols] block of a row-major array into LDS: `issue`
// loads up to P pieces per thread into registers, `commit` writes them. Loads issued
// before the weight batch can be committed without waiting for the weights.
template <typename T, int P>
struct Staged {
  T v[P];
  int n;  // pieces this thread loaded
};

template <typename T, int P>
__device__ inline void stage_issue(Staged<T, P>& st, const T* src, int64_t ld, int rows, int cols, int first) {
  st.n = 0;
#pragma unroll
  for (int j = 0; j < P; ++j) {
    const int i = first + threadIdx.x + j * blockDim.x;
    if (i < rows * cols) {
      const int rr = i / cols, c = i - rr * cols;
      st.v[j] = src[rr * ld + c];
      st.n = j + 1;
    }
  }
}

template <typename T, int P>
__device__ inline void stage_commit(const Staged<T, P>& st, T* dst, int ldd, int rows, int cols, int first) {
#pragma unroll
  for (int j = 0; j < P; ++j) {
    const int i = first + threadIdx.x + j * blockDim.x;
    if (j < st.n) {
      const int rr = i / cols, c = i - rr * cols;
      dst[rr * ldd + c] = st.v[j];
    }
  }
}

// Weights of U consecutive k-steps for NT row tiles.
template <int KIND, int NT, int UB = 16>
struct Batch {
  static constexpr int NL = KIND == KIND_INT4 ? 1 : 2;
  static constexpr int U = batch_steps<KIND, NT, UB>();
  uint4 w[U][NT][NL];
};

// Every load is issued (k-steps past kend re-read the last valid one, an L2 hit) so the
// number of loads in flight is static and the compiler can wait for exactly the batch
// it consumes.
template <int KIND, int NT, int UB>
__device__ inline void load_batch(const uint8_t* const* wrow, Batch<KIND, NT, UB>& bt, int kst0, int kend, int g) {
  using B = Batch<KIND, NT, UB>;
#pragma unroll
  for (int u = 0; u < B::U; ++u) {
    const int kst = min(kst0 + u, kend - 1);
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int L = 0; L < B::NL; ++L) bt.w[u][t][L] = load_nt16(wrow[t] + w_off<KIND>(kst, g, L));
  }
}

// Multiply one batch: activations of k-step kst at LDS column (kst - chunk0) * 128, rows
// 16 mt + r; rows >= M re-read row M - 1 (MFMA rows are independent and those outputs
// are discarded). acc: scaled result (int4) or raw sum x * (128 + q) (int8); accg: int4
// current group. The sum of x over each group (for the 128 offset) comes from q.xsum.
template <int KIND, int MT, int NT, bool HZ, int SD, int UB>
__device__ inline void compute_batch(const GroupQ<SD>& q, int M, const Batch<KIND, NT, UB>& bt, const uint16_t* lds,
                                     int lds_stride, int kst0, int kend, int chunk0, int r, int g,
                                     f32x4 (&acc)[NT][MT], f32x4 (&accg)[NT][MT]) {
  using B = Batch<KIND, NT, UB>;
  const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int u = 0; u < B::U; ++u) {
    const int kst = kst0 + u;
    if (kst < kend) {  // a guard, not a break: the loop must unroll fully (register arrays)
    const int kl = kst - chunk0;
    bf16x8 a[MT][4];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const uint16_t* row = lds + min(mt * 16 + r, M - 1) * lds_stride;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint4 v = *reinterpret_cast<const uint4*>(row + a_off<KIND>(kl, g, j));
        a[mt][j] = as_bf16x8(v.x, v.y, v.z, v.w);
      }
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      bf16x8 b[4];
      unpack_b<KIND>(bt.w[u][t], b);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (KIND == KIND_INT4) accg[t][mt] = mfma(a[mt][j], b[j], accg[t][mt]);
          else acc[t][mt] = mfma(a[mt][j], b[j], acc[t][mt]);
        }
    }
    if (KIND == KIND_INT4 && (kst + 1) % q.group_steps == 0) {  // end of a quantization group
      const int gl = kst / q.group_steps - q.g0;
      f32x4 xs[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        xs[mt] = *reinterpret_cast<const f32x4*>(q.xsum + gl * q.xrows + mt * 16 + g * 4);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int si = (t * 16 + r) * q.stride + gl;
        const float sc = sd_to_f32<SD>(q.sc[si]);
        const float cz = HZ ? sd_to_f32<SD>(q.zr[si]) - 128.f * sc : -136.f * sc;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
          for (int v = 0; v < 4; ++v) acc[t][mt][v] += sc * accg[t][mt][v] + cz * xs[mt][v];
          accg[t][mt] = z4;
        }
      }
    }
    }
  }
}

// Sums of the staged activations over each k-step of 128 (rows < M, local k-steps
// [0, nsteps)), added into xsum[slot(kl) * xrows + m] with LDS atomics; slot = the
// group index for int4, 0 for int8 (the whole range). xsum must be zeroed first.
__device__ inline void sum_activations(const uint16_t* lds, int lds_stride, int M, int nsteps, int kst_first,
                                       int group_steps, int g0, bool per_group, float* xsum, int xrows) {
  for (int i = threadIdx.x; i < M * nsteps; i += blockDim.x) {
    const int m = i / nsteps, kl = i - m * nsteps;
    const uint16_t* p = lds + m * lds_stride + kl * kStepK;
    float s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int c = 0; c < kStepK / 8; ++c) {
      const uint4 v = *reinterpret_cast<const uint4*>(p + c * 8);
      s0 += bf16_to_f32(v.x & 0xffff) + bf16_to_f32(v.y & 0xffff) + bf16_to_f32(v.z & 0xffff) + bf16_to_f32(v.w & 0xffff);
      s1 += bf16_to_f32(v.x >> 16) + bf16_to_f32(v.y >> 16) + bf16_to_f32(v.z >> 16) + bf16_to_f32(v.w >> 16);
    }
    const int slot = per_group ? (kst_first + kl) / group_steps - g0 : 0;
    atomicAdd(xsum + slot * xrows + m, s0 + s1);
  }
}

// Stream k-steps [a, b) of NT row tiles with the next batch of weights in flight while
// the current one is unpacked and multiplied. `first` must already hold the batch
// starting at a (issued before the activation staging).
template <int KIND, int MT, int NT, bool HZ, int SD, int UB>
__device__ inline void stream_steps(const GroupQ<SD>& q, int M, const uint8_t* const* wrow,
                                    Batch<KIND, NT, UB>& first, const uint16_t* lds, int lds_stride, int a, int b,
                                    int chunk0, int r, int g, f32x4 (&acc)[NT][MT], f32x4 (&accg)[NT][MT]) {
  using B = Batch<KIND, NT, UB>;
  Batch<KIND, NT, UB> other;
  for (int k = a; k < b;) {
    const int k2 = k + B::U;
    if (k2 < b) load_batch<KIND, NT, UB>(wrow, other, k2, b, g);
    compute_batch<KIND, MT, NT, HZ, SD, UB>(q, M, first, lds, lds_stride, k, b, chunk0, r, g, acc, accg);
    if (k2 >= b) break;
    const int k3 = k2 + B::U;
    if (k3 < b) load_batch<KIND, NT, UB>(wrow, first, k3, b, g);
    compute_batch<KIND, MT, NT, HZ, SD, UB>(q, M, other, lds, lds_stride, k2, b, chunk0, r, g, acc, accg);
    k = k3;
  }
}

}  // namespace wo
}  // namespace miq
