// Weight-only quantized GEMM for long prefill chunks (large M), gfx950:
//
//   y[m, n] = sum_k x[m, k] * W[n, k],  x bf16 [M, K],  W int8 [N, K] or int4 [N, K/2]
//
// A workgroup of 4 wavefronts (one per SIMD) owns 128 weight rows x 128 MT activation rows;
// wavefront w owns activation rows 32 MT w .. 32 MT w + 32 MT - 1 against all 128 weight
// rows (4 MT accumulator tiles of 32 x 32 in AGPRs). Per 128-k step the workgroup
// dequantizes its 128 x 128 weight block once, into LDS, as bf16 MFMA operand fragments:
//   int4: the reference's weight, bit for bit: bf16(SD(SD(q s) + z)) in the scale dtype SD's
//         arithmetic (symmetric codes: bf16(SD((q - 8) s))), 3 to 5 VALU instructions per
//         code;
//   int8: w = q, exact in bf16; the per-row scale is applied to the output as int8_wo does,
//         y = bf16(bf16(acc) * bf16(s)).
// The dequantize work (about 23 (symmetric) to 43 (zero points) VALU instructions per 8
// int4 codes, 8 codes per thread and sub-step) is done once per workgroup and feeds 4 MT MFMAs per fragment per wavefront
// (the decode-shaped prefill kernel instead unpacks the weights in every wavefront and
// corrects the +128 code offset with per-group activation sums: about 7 VALU instructions
// per MFMA, which bounds it well below the MFMA peak at large M).
//
// The activations are first packed (wo_wide_pack_kernel) into operand order: every load
// of the main kernel is then 1 KiB of contiguous memory. Loaded straight from x, each load
// touched 32 rows 16-32 bytes at a time and the texture units, stalled on L1 tag
// conflicts, set the pace. The packed copy sits in the caller's workspace and is cleared
// again afterwards (wo_wide_clear_kernel), because the decode kernels rely on that
// workspace being zero between calls.
//
// MFMA: v_mfma_f32_32x32x16_bf16 (weights as the A operand, 32 rows; activations as the B
// operand, 32 rows). Sub-step c (0..7) of a k-step takes k = 16 c + 8 (l / 32) + e,
// e = 0..7, in lane l; the weight fragment of (c, tile t) is 64 consecutive 16-byte LDS
// slots, read with asm ds_read_b128 one sub-step ahead and waited for explicitly (the
// compiler otherwise sank every read next to its first use, exposing the LDS latency to
// the one wavefront of the SIMD). A 32 x 32 tile leaves each lane four consecutive outputs
// of one activation row per group of four accumulators: one 8-byte store.
#include <algorithm>
#include <type_traits>

#include "miq_common.h"
#include "wo_core.h"
#include "wo_wide.h"

namespace miq {
namespace {

using namespace wo;

constexpr int kWN = 128;                // weight rows per workgroup
constexpr int kWNT = kWN / 32;          // 32-row weight tiles per workgroup
constexpr int kWBuf = kWN * kStepK;     // bf16 elements of one dequantized k-step
constexpr int kOutW = 0x7ffffff0;       // outside every buffer: the load returns zeros

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

struct WideParams {
  const uint16_t* x;    // the packed activations
  const uint8_t* w;
  int64_t ldw;          // bytes per weight row
  const void* scale;
  const void* zero;
  int group_steps;      // int4: k-steps per quantization group
  int64_t ngroups;      // int4: groups per weight row
  uint16_t* y;
  int64_t ldy;
  int M, N, steps;      // steps = K / 128
  int tiles_m, tiles_n;
  int xbytes, wbytes, sbytes;  // bytes of the packed activations, weights, scales
  bool vec_store;       // y 8-byte aligned with ldy % 4 == 0
  bool m_major;         // tiles ordered activation panel by activation panel
  int S, split_steps;   // K splits and k-steps per split
  float* part;          // S > 1: S fp32 partial outputs [M][N], split_stride floats apart
  int64_t split_stride;
};

// f(integral_constant<int, 0>) ... f(integral_constant<int, N - 1>), in order
template <int N, int I = 0, class F>
__device__ inline void unroll_r(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    unroll_r<N, I + 1>(f);
  }
}

typedef __attribute__((address_space(3))) uint16_t lds_u16;

// 16-byte LDS read at a compile-time offset from `addr` (an LDS byte address). Issued as asm
// so that the compiler cannot sink it next to its use: the caller waits for it explicitly
// with lds_wait, which also carries the data dependence to the MFMAs.
template <int OFF>
__device__ inline bf16x8 lds_read16(uint32_t addr) {
  bf16x8 r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
  return r;
}

// Waits until at most N LDS operations are outstanding; the 4 fragments pass through the
// statement, so nothing that uses them is scheduled before it. LDS operations complete in
// order, so with the 4 reads issued after them still in flight (N = 4) the fragments are in.
template <int N>
__device__ inline void lds_wait(bf16x8 (&b)[4]) {
  asm volatile("s_waitcnt lgkmcnt(%4)" : "+v"(b[0]), "+v"(b[1]), "+v"(b[2]), "+v"(b[3]) : "i"(N));
}

__device__ inline uint32_t pack_bf16x2(float a, float b) {
  const bf16x2_t v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
  return __builtin_bit_cast(uint32_t, v);
}

// The two bf16 values of a packed pair, widened to fp32 (exact).
__device__ inline float bf16_lo(uint32_t p) { return __builtin_bit_cast(float, p << 16); }
__device__ inline float bf16_hi(uint32_t p) { return __builtin_bit_cast(float, p & 0xffff0000u); }

// The reference's dequantized int4 weight (int4_wo.py:33-42 and its symmetric form), for
// codes q (as fp32), computed in the scale dtype's arithmetic (each op rounded to it, as
// torch does on the CPU) and then rounded to bf16 for the matmul, as
// QuantMethod.linear's .to(x.dtype) does (base.py:20-24), so the weights are the
// reference's bit for bit:
//   zero points:  w = bf16(SD(SD(q s) + z));   symmetric: w = bf16(SD((q - 8) s)),
// with z = -8 s passed for the symmetric form. q s is exact in fp32 for bf16 / f16 scales.
template <int SD, bool HZ>
__device__ inline uint32_t dequant_pair(float q0, float q1, float s, float z) {
  if constexpr (!HZ) {
    // (q - 8) s = fma(q, s, -8 s), rounded once to fp32 (exact for bf16 / f16 scales)
    float a = __builtin_fmaf(q0, s, z), b = __builtin_fmaf(q1, s, z);
    if constexpr (SD == MIQ_F16) {
      a = static_cast<float>(static_cast<_Float16>(a));
      b = static_cast<float>(static_cast<_Float16>(b));
    }
    return pack_bf16x2(a, b);
  } else if constexpr (SD == MIQ_BF16) {
    const uint32_t p = pack_bf16x2(q0 * s, q1 * s);  // bf16(q s), q s exact in fp32
    return pack_bf16x2(bf16_lo(p) + z, bf16_hi(p) + z);
  } else if constexpr (SD == MIQ_F16) {
    const float a = static_cast<float>(static_cast<_Float16>(q0 * s));
    const float b = static_cast<float>(static_cast<_Float16>(q1 * s));
    return pack_bf16x2(static_cast<float>(static_cast<_Float16>(a + z)),
                       static_cast<float>(static_cast<_Float16>(b + z)));
  } else {
    // fp32: the product and the sum each rounded; the empty asm statement keeps the
    // compiler from contracting them into one fma
    float a = q0 * s, b = q1 * s;
    asm("" : "+v"(a), "+v"(b));
    return pack_bf16x2(a + z, b + z);
  }
}

// 8 int4 codes of one word (low nibble first) -> the 8 reference weights, natural k order.
// The masked words pass through an empty asm statement so that the byte converts stay
// v_cvt_f32_ubyte{0..3} on the masked words (otherwise each nibble becomes its own
// bitfield extract).
template <int SD, bool HZ>
__device__ inline uint4 dequant_u4(uint32_t w, float s, float z) {
  uint32_t lo = w & 0x0f0f0f0fu, hi = (w >> 4) & 0x0f0f0f0fu;
  asm volatile("" : "+v"(lo), "+v"(hi));
  uint4 o;
  o.x = dequant_pair<SD, HZ>(static_cast<float>(lo & 0xffu), static_cast<float>(hi & 0xffu), s, z);
  o.y = dequant_pair<SD, HZ>(static_cast<float>((lo >> 8) & 0xffu), static_cast<float>((hi >> 8) & 0xffu), s, z);
  o.z = dequant_pair<SD, HZ>(static_cast<float>((lo >> 16) & 0xffu), static_cast<float>((hi >> 16) & 0xffu), s, z);
  o.w = dequant_pair<SD, HZ>(static_cast<float>(lo >> 24), static_cast<float>(hi >> 24), s, z);
  return o;
}

// 8 int8 codes (two words) -> 8 bf16 values of the signed codes (exact)
__device__ inline uint4 dequant_i8(uint32_t w0, uint32_t w1) {
  uint4 o;
  o.x = pack_bf16x2(static_cast<float>(static_cast<int8_t>(w0)), static_cast<float>(static_cast<int8_t>(w0 >> 8)));
  o.y = pack_bf16x2(static_cast<float>(static_cast<int8_t>(w0 >> 16)), static_cast<float>(static_cast<int8_t>(w0 >> 24)));
  o.z = pack_bf16x2(static_cast<float>(static_cast<int8_t>(w1)), static_cast<float>(static_cast<int8_t>(w1 >> 8)));
  o.w = pack_bf16x2(static_cast<float>(static_cast<int8_t>(w1 >> 16)), static_cast<float>(static_cast<int8_t>(w1 >> 24)));
  return o;
}

template <int KIND, bool HZ, int SD, int MT>
__global__ void __launch_bounds__(256, 1)
wo_wide_kernel(WideParams p) {
  constexpr bool I4 = KIND == KIND_INT4;
  constexpr int WL = I4 ? 2 : 4;       // 16-byte weight loads per thread and k-step
  constexpr int WSTEP = I4 ? 64 : 128; // weight bytes per row and k-step
  constexpr int esz = SD == MIQ_F32 ? 4 : 2;
  __shared__ __align__(16) uint16_t s_w[2][kWBuf];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;

  // tile of this workgroup: XCD x (= id % 8) takes tiles [x T / 8, (x + 1) T / 8), weight
  // panel by weight panel (all activation tiles of a panel in a row) or, with m_major,
  // activation panel by activation panel, so that the workgroups that read the same operand
  // block run on one XCD and share its L2; the launcher orders by the larger operand
  const int T = p.tiles_m * p.tiles_n, I = T * p.S;
  const int xcd = blockIdx.x & 7, local = blockIdx.x >> 3;
  const int item = (int)((int64_t)I * xcd / 8) + local;
  if (item >= (int)((int64_t)I * (xcd + 1) / 8)) return;
  // item = split * T + tile: XCDs take contiguous blocks of items, so an XCD's workgroups
  // share one split's K range of the weights and activations
  const int split = item / T, tile = item - split * T;
  const int sb = split * p.split_steps, s_end = min(p.steps, sb + p.split_steps);  // this split's k-steps
  int tn, tm;
  if (p.m_major) {
    tm = tile / p.tiles_n;
    tn = tile - tm * p.tiles_n;
  } else {
    tn = tile / p.tiles_m;
    tm = tile - tn * p.tiles_m;
  }
  const int n0 = tn * kWN, mw = (tm * 4 + wv) * 32 * MT;

  // ---- weights: thread -> row wr = 16 (tid / 32) + tid % 16 of the block, half wh of the
  // step's bytes (int4: 32 of 64, int8: 64 of 128), 64 codes = 8 chunks of 8 k
  const int wr = 16 * (tid >> 5) + (tid & 15), wh = (tid >> 4) & 1;
  const bool wok = n0 + wr < p.N;
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(p.w), 0, p.wbytes, 0x00020000);
  const int wbase = (n0 + wr) * (int)p.ldw + wh * (WSTEP / 2);
  const __amdgpu_buffer_rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p.scale), 0, p.sbytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t zrs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(HZ ? p.zero : p.scale), 0, p.sbytes, 0x00020000);
  const int64_t srow = (int64_t)min(n0 + wr, p.N - 1) * p.ngroups;
  // LDS slot of chunk q (k = 64 wh + 8 q): sub-step c = 4 wh + q / 2, lane half q % 2,
  // tile t = wr / 32, lane wr % 32 + 32 (q % 2). The 16 threads of each write phase hold
  // 16 consecutive rows: 256 contiguous bytes, no bank conflicts.
  auto w_slot = [&](int q) {
    return (((4 * wh + (q >> 1)) * kWNT + (wr >> 5)) * 64 + (wr & 31) + 32 * (q & 1)) * 8;
  };

  uint4 wreg[2][WL];
  uint32_t sw[2], zw[2];
  auto load_w = [&](auto set_c, int s) {
    constexpr int set = decltype(set_c)::value;
    const int off = wok && s < s_end ? wbase + s * WSTEP : kOutW;
#pragma unroll
    for (int l = 0; l < WL; ++l) {
      const auto v = __builtin_amdgcn_raw_buffer_load_b128(wrs, off, 16 * l, 0);
      wreg[set][l] = *reinterpret_cast<const uint4*>(&v);
    }
    if constexpr (I4) {
      const int gi = (int)(srow + min(s, p.steps - 1) / p.group_steps);
      sw[set] = __builtin_amdgcn_raw_buffer_load_b32(srs, (gi * esz) & ~3, 0, 0);
      zw[set] = HZ ? __builtin_amdgcn_raw_buffer_load_b32(zrs, (gi * esz) & ~3, 0, 0) : 0u;
    }
  };
  // chunk q of the weights in register set `set`, dequantized
  auto dequant_chunk = [&](auto set_c, int q, float sc, float zz) {
    constexpr int set = decltype(set_c)::value;
    if constexpr (I4) {
      const uint4& wv4 = wreg[set][q >> 2];
      const uint32_t d = (q & 3) == 0 ? wv4.x : (q & 3) == 1 ? wv4.y : (q & 3) == 2 ? wv4.z : wv4.w;
      return dequant_u4<SD, HZ>(d, sc, zz);
    } else {
      const uint4& wv4 = wreg[set][q >> 1];
      return (q & 1) ? dequant_i8(wv4.z, wv4.w) : dequant_i8(wv4.x, wv4.y);
    }
  };
  // this step's scale and zero of the thread's weight row (int4)
  auto group_sz = [&](auto set_c, int s, float& sc, float& zz) {
    constexpr int set = decltype(set_c)::value;
    if constexpr (I4) {
      const int gi = (int)(srow + min(s, p.steps - 1) / p.group_steps);
      sc = word_to_f32<SD>(sw[set], gi);
      zz = HZ ? word_to_f32<SD>(zw[set], gi) : -8.f * sc;
    }
  };

  // ---- activations, packed by wo_wide_pack_kernel: fragment (32-row tile r, step s,
  // sub-step c) is 1 KiB at ((r * steps + s) * 8 + c) KiB, lane l's 16 bytes at 16 l (rows
  // l % 32 of the tile, k = 128 s + 16 c + 8 (l / 32) .. + 7), so every load is 1 KiB of
  // contiguous memory
  const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(p.x), 0, p.xbytes, 0x00020000);
  int xoff[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) xoff[i] = ((mw >> 5) + i) * p.steps * 8192 + lane * 16;
  bf16x8 a[2][MT][8];
  // the activations of sub-step c of step s into set `set`
  auto load_a = [&](auto set_c, int s, int c) {
    constexpr int set = decltype(set_c)::value;
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      const int off = s < s_end ? xoff[i] + s * 8192 : kOutW;
      const auto v = __builtin_amdgcn_raw_buffer_load_b128(xrs, off, 1024 * c, 0);
      a[set][i][c] = __builtin_bit_cast(bf16x8, v);
    }
  };
  // this lane's slot in LDS buffer 0 (fragment (c, t) is 1 KiB further per (c, t), buffer 1
  // 32 KiB further)
  const uint32_t lds_lane = (uint32_t)(size_t)(lds_u16*)&s_w[0][0] + lane * 16;

  f32x16 acc[MT][kWNT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int t = 0; t < kWNT; ++t)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][t][v] = 0.f;

  // One k-step: multiply dequantized buffer `buf` with activation set `aset` while the
  // weights of the next step (register set `wset`) are dequantized into the other buffer,
  // one chunk per sub-step. Sub-step c requests the activations of sub-step c of the next
  // step and the weight fragments of sub-step c + 1 (asm LDS reads, waited for explicitly
  // one sub-step later), then issues its 4 MT MFMAs.
  auto step = [&](auto aset_c, auto wset_c, auto buf_c, int s) {
    constexpr int aset = decltype(aset_c)::value, buf = decltype(buf_c)::value;
    // the loaded weight words pass through an empty volatile asm statement here, so that no
    // arithmetic on them is hoisted into the previous step (where it would wait for loads
    // issued in that same step)
    constexpr int wset = decltype(wset_c)::value;
#pragma unroll
    for (int l = 0; l < WL; ++l)
      asm volatile("" : "+v"(wreg[wset][l].x), "+v"(wreg[wset][l].y), "+v"(wreg[wset][l].z), "+v"(wreg[wset][l].w));
    if constexpr (I4) asm volatile("" : "+v"(sw[wset]), "+v"(zw[wset]));
    float sc = 0.f, zz = 0.f;
    group_sz(wset_c, s + 1, sc, zz);
    uint16_t* dst = s_w[buf ^ 1];
    constexpr int bo = buf * kWBuf * 2;  // byte offset of the buffer
    bf16x8 b[2][kWNT];
    unroll_r<kWNT>([&](auto t_c) { b[0][decltype(t_c)::value] = lds_read16<bo + decltype(t_c)::value * 1024>(lds_lane); });
    unroll_r<8>([&](auto c_c) {
      constexpr int c = decltype(c_c)::value;
      load_a(std::integral_constant<int, aset ^ 1>{}, s + 1, c);
      if constexpr (c < 7) {
        unroll_r<kWNT>([&](auto t_c) {
          constexpr int t = decltype(t_c)::value;
          b[(c + 1) & 1][t] = lds_read16<bo + ((c + 1) * kWNT + t) * 1024>(lds_lane);
        });
        lds_wait<kWNT>(b[c & 1]);
      } else {
        lds_wait<0>(b[c & 1]);
      }
      *reinterpret_cast<uint4*>(dst + w_slot(c)) = dequant_chunk(wset_c, c, sc, zz);
#pragma unroll
      for (int t = 0; t < kWNT; ++t)
#pragma unroll
        for (int i = 0; i < MT; ++i)
          acc[i][t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b[c & 1][t], a[aset][i][c], acc[i][t], 0, 0, 0);
    });
  };

  // Two register sets and LDS buffers, over the split's k-steps sb .. s_end - 1. Step s
  // multiplies buffer (s - sb) % 2 with activation set (s - sb) % 2 while the weights of
  // step s + 1 are dequantized into the other buffer; it requests
  // the weights of step s + 2 when it starts and the activations of sub-step c of step s + 1
  // at its sub-step c, so each request has a whole step to arrive and only one step of
  // activations occupies registers at a time. Steps past the end read zeros (activations)
  // and add nothing.
  constexpr auto C0 = std::integral_constant<int, 0>{};
  load_w(C0, sb);
  load_w(std::integral_constant<int, 1>{}, sb + 1);
#pragma unroll
  for (int c = 0; c < 8; ++c) load_a(C0, sb, c);
  {
    float sc = 0.f, zz = 0.f;
    group_sz(C0, sb, sc, zz);
#pragma unroll
    for (int q = 0; q < 8; ++q) *reinterpret_cast<uint4*>(s_w[0] + w_slot(q)) = dequant_chunk(C0, q, sc, zz);
  }
  __syncthreads();
  for (int s0 = sb; s0 < s_end; s0 += 2) {
    unroll_r<2>([&](auto ph_c) {
      constexpr int ph = decltype(ph_c)::value;
      const int s = s0 + ph;
      load_w(ph_c, s + 2);
      step(ph_c, std::integral_constant<int, ph ^ 1>{}, ph_c, s);
      __syncthreads();
    });
  }

  // ---- epilogue: acc[i][t][4 g + v] = y[mw + 32 i + lane % 32][n0 + 32 t + 8 g + 4 (lane / 32) + v]
  if (p.S > 1) {
    // split K: this split's fp32 partial tile; wo_wide_reduce_kernel adds the splits
    float* part = p.part + (int64_t)split * p.split_stride;
#pragma unroll
    for (int t = 0; t < kWNT; ++t)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = n0 + 32 * t + 8 * g + 4 * (lane >> 5);
        if (n >= p.N) continue;
#pragma unroll
        for (int i = 0; i < MT; ++i) {
          const int m = mw + 32 * i + (lane & 31);
          if (m >= p.M) continue;
          float* dst = part + (int64_t)m * p.N + n;
          if ((p.N & 3) == 0) {
            *reinterpret_cast<float4*>(dst) =
                make_float4(acc[i][t][4 * g], acc[i][t][4 * g + 1], acc[i][t][4 * g + 2], acc[i][t][4 * g + 3]);
          } else {
#pragma unroll
            for (int v = 0; v < 4; ++v)
              if (n + v < p.N) dst[v] = acc[i][t][4 * g + v];
          }
        }
      }
    return;
  }
#pragma unroll
  for (int t = 0; t < kWNT; ++t)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int n = n0 + 32 * t + 8 * g + 4 * (lane >> 5);
      if (n >= p.N) continue;  // N is a multiple of 16: the 4 outputs are all in range
      float rs[4] = {1.f, 1.f, 1.f, 1.f};
      if constexpr (!I4) {
#pragma unroll
        for (int v = 0; v < 4; ++v) rs[v] = bf16_to_f32(f32_to_bf16(sd_to_f32<SD>(load_sd_raw<SD>(p.scale, n + v))));
      }
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        const int m = mw + 32 * i + (lane & 31);
        if (m >= p.M) continue;
        float o[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float f = acc[i][t][4 * g + v];
          o[v] = I4 ? f : bf16_to_f32(f32_to_bf16(f)) * rs[v];
        }
        uint16_t* dst = p.y + (int64_t)m * p.ldy + n;
        if (p.vec_store) {
          *reinterpret_cast<uint2*>(dst) = make_uint2(pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3]));
        } else {
#pragma unroll
          for (int v = 0; v < 4; ++v) dst[v] = f32_to_bf16(o[v]);
        }
      }
    }
}

// Packs x [M, K] (bf16, row stride ldx) into the wide kernel's operand order: workgroup
// (tile r of 32 rows, k-step s) reads the tile's 32 x 128 block with coalesced 16-byte loads
// (rows past M read as zeros), transposes it through LDS and writes its 8 fragments as 8 KiB
// of contiguous memory.
__global__ void __launch_bounds__(256) wo_wide_pack_kernel(const uint16_t* __restrict__ x, int64_t ldx, int M,
                                                           int steps, uint16_t* __restrict__ out) {
  __shared__ __align__(16) uint4 s_t[512];
  const int r = blockIdx.y, s = blockIdx.x, tid = threadIdx.x;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int piece = tid + 256 * j, row = piece >> 4, ch = piece & 15, m = 32 * r + row;
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (m < M) v = *reinterpret_cast<const uint4*>(x + (int64_t)m * ldx + (int64_t)s * kStepK + 8 * ch);
    // fragment c = ch / 2, lane row + 32 (ch % 2)
    s_t[(ch >> 1) * 64 + row + 32 * (ch & 1)] = v;
  }
  __syncthreads();
  uint4* dst = reinterpret_cast<uint4*>(out) + ((int64_t)r * steps + s) * 512;
#pragma unroll
  for (int j = 0; j < 2; ++j) dst[tid + 256 * j] = s_t[tid + 256 * j];
}

// Writes zeros over n16 16-byte words (the packed activations, so that the workspace is all
// zeros again when the call ends).
__global__ void __launch_bounds__(256) wo_wide_clear_kernel(i32x4* __restrict__ p, int64_t n16) {
  const i32x4 z = {0, 0, 0, 0};
  const int64_t i = (int64_t)blockIdx.x * 1024 + threadIdx.x;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (i + 256 * j < n16) p[i + 256 * j] = z;
}

// y = the sum of the S partial outputs of a split launch, in split order (the same sum
// whichever workgroup finishes first), for int8 rounded to bf16 and scaled as the
// unsplit epilogue does; the partials are overwritten with zeros (the workspace is zero
// between calls). A thread takes 4 consecutive elements of the flattened [M][N] output
// (16-byte loads: split_stride is a multiple of 4).
// The packed activations are cleared by the same launch: its first clear_blocks workgroups
// run wo_wide_clear_kernel's work, the others the reduction.
template <bool I8, int SD>
__global__ __launch_bounds__(256) void wo_wide_reduce_kernel(float* part, int64_t split_stride, int S, int M, int N,
                                                             const void* scale, uint16_t* y, int64_t ldy,
                                                             i32x4* pack, int64_t n16, int clear_blocks) {
  if ((int)blockIdx.x < clear_blocks) {
    const i32x4 z = {0, 0, 0, 0};
    const int64_t i = (int64_t)blockIdx.x * 1024 + threadIdx.x;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (i + 256 * j < n16) pack[i + 256 * j] = z;
    return;
  }
  const int64_t e = ((int64_t)(blockIdx.x - clear_blocks) * 256 + threadIdx.x) * 4;
  const int64_t MN = (int64_t)M * N;
  if (e >= MN) return;
  float4 sum = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int s0 = 0; s0 < S; s0 += 4) {
    float4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u)
      v[u] = s0 + u < S ? *reinterpret_cast<const float4*>(part + (s0 + u) * split_stride + e)
                        : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (s0 + u < S) *reinterpret_cast<float4*>(part + (s0 + u) * split_stride + e) = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      sum.x += v[u].x;
      sum.y += v[u].y;
      sum.z += v[u].z;
      sum.w += v[u].w;
    }
  }
  const float o[4] = {sum.x, sum.y, sum.z, sum.w};
  int m = (int)(e / N), n = (int)(e - (int64_t)m * N);
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    if (e + v >= MN) break;
    float val = o[v];
    if constexpr (I8) val = bf16_to_f32(f32_to_bf16(val)) * bf16_to_f32(f32_to_bf16(sd_to_f32<SD>(load_sd_raw<SD>(scale, n))));
    y[(int64_t)m * ldy + n] = f32_to_bf16(val);
    if (++n == N) {
      n = 0;
      ++m;
    }
  }
}

template <int KIND, bool HZ, int SD, int MT>
void launch_wide(const WideParams& p, hipStream_t st) {
  const unsigned items = (unsigned)(p.tiles_m * p.tiles_n * p.S);
  const unsigned grid = (items + 7) / 8 * 8 + 8;  // every XCD block fits its share
  hipLaunchKernelGGL((wo_wide_kernel<KIND, HZ, SD, MT>), dim3(grid), dim3(256), 0, st, p);
}

}  // namespace

// Bytes of the fp32 partial outputs of a launch with S > 1 K splits (0 for S = 1).
size_t wo_wide_part_bytes(int64_t M, int64_t N, int S) {
  return S > 1 ? (size_t)S * (size_t)((M * N + 3) & ~3LL) * 4 : 0;
}

// Bytes of the packed activations of a call (32-row tiles of whole workgroups).
size_t wo_wide_pack_bytes(int64_t M, int64_t K, int mt) {
  const int64_t tiles_m = (M + 128 * mt - 1) / (128 * mt);
  return (size_t)(tiles_m * 4 * mt * 32) * (size_t)K * 2;
}

// Plan of a call: activation tiles per wavefront (mt, 1..3; 0 = the wide kernel would leave
// most CUs idle, so the prefill kernel, whose smaller tiles fill the GPU, runs instead) and
// K splits (S). A launch of T tiles and S splits is T S workgroups in ceil(T S / 256) rounds
// (one per CU), each as long as MT 32-row tiles over ceil(steps / S) k-steps (rounded up to
// an even count: the loop takes steps in pairs). The modelled time is
//   0.8 us * rounds * MT * c(MT) * k-steps  +  0.5 us per MB of fp32 partials (S > 1)
// with c = 1.75, 1.13, 1.0 for MT = 1, 2, 3, fitted on MI355X to a sweep of every MT and
// S = 1 .. 16 (N x K = 2560 x 9728, 4096 x 4096, 2560 x 2560, 6144 x 4096, 4096 x 12288;
// M = 65 .. 4096), where the plan of least modelled time came within 1 % of the fastest on
// average. The plan of least modelled time is taken (the larger MT, then the fewer splits,
// on ties); plans below 128 workgroups (half the CUs) are not taken unless MT is forced
// (MIQ_WO_WIDE_MT). Splits are planned only from 48 k-steps (K >= 6144) up: at shorter K
// the pack, reduce and clear launches around a short split launch cost more than the
// prefill kernel does (2560 x 2560 at M = 128 .. 768: 23-41 us split against 22-34 us),
// while at K = 9728 and 12288 the split launch beats it by 10-35 % from M = 65 up. The plan
// does not depend on the workspace a call brings: a call whose workspace cannot hold it
// runs the prefill kernel instead.
WidePlan wo_wide_plan(int64_t M, int64_t N, int64_t K, int64_t ldw) {
  static const double kCost[4] = {0.0, 1.75, 1.13, 1.0};
  constexpr int64_t kMinSplitSteps = 48;
  const int forced_mt = tuning().wo_wide_mt, forced_s = tuning().wo_wide_s;
  const int64_t tiles_n = (N + kWN - 1) / kWN, steps = K / kStepK;
  const int max_s = forced_s >= 1 || steps >= kMinSplitSteps ? 16 : 1;
  WidePlan best{};
  double best_t = 0.0;
  for (int mt = 1; mt <= 3; ++mt) {
    if (forced_mt >= 1 && forced_mt <= 3 && mt != forced_mt) continue;
    const size_t pack = wo_wide_pack_bytes(M, K, mt);
    if (pack >= 0x7fff0000ULL || N * ldw >= 0x7fff0000LL) continue;
    const int64_t tiles = (M + 128 * mt - 1) / (128 * mt) * tiles_n;
    for (int S = 1; S <= max_s; ++S) {
      const int64_t per = (steps + S - 1) / S;
      if ((steps + per - 1) / per != S) continue;  // no empty splits
      if (forced_s >= 1) {  // MIQ_WO_WIDE_S (at most 16 and steps), less any empty splits
        const int64_t fs = std::min<int64_t>(std::min(forced_s, 16), steps);
        if (per != (steps + fs - 1) / fs) continue;
      }
      const size_t part = wo_wide_part_bytes(M, N, S);
      const int64_t items = tiles * S;
      if (items < 128 && forced_mt < 1) continue;
      const double t = 0.8 * (double)((items + 255) / 256) * mt * kCost[mt] * (double)((per + 1) & ~1LL) +
                       (double)part * 0.5e-6;
      if (best.mt == 0 || t < best_t - 1e-9 || (t <= best_t + 1e-9 && mt > best.mt)) {
        best.mt = mt;
        best.S = S;
        best.split_steps = (int)per;
        best.pack_bytes = pack;
        best.part_bytes = part;
        best_t = t;
      }
    }
  }
  return best;
}

// Launches the wide path: pack the activations into the first pl.pack_bytes of `ws` (zero on
// entry), run the kernel (with pl.S > 1 it writes fp32 partial outputs after the packed
// activations, and the reduce kernel adds them into y and clears them), and clear the packed
// activations again (in the reduce kernel's launch when there is one), so `ws` is zero
// afterwards. Returns a MIQ_* status.
int wo_wide_launch(int kind, const WidePlan& pl, const uint16_t* x, int64_t ldx, const uint8_t* w, int64_t ldw,
                   const void* scale, const void* zero, int sd, int group_steps, int64_t ngroups, uint16_t* y,
                   int64_t ldy, int64_t M, int N, int K, void* ws, size_t ws_bytes, hipStream_t st,
                   const char* name) {
  const int mt = pl.mt;
  MIQ_REQUIRE(mt >= 1 && mt <= 3 && pl.S >= 1 && pl.pack_bytes == wo_wide_pack_bytes(M, K, mt) &&
                  pl.pack_bytes < 0x7fff0000ULL && (int64_t)N * ldw < 0x7fff0000LL,
              "%s: operands too large for the wide kernel", name);
  const size_t need = pl.pack_bytes + pl.part_bytes;
  MIQ_REQUIRE(ws != nullptr && ws_bytes >= need && (reinterpret_cast<uintptr_t>(ws) & 15) == 0,
              "%s: the wide kernel needs %zu bytes of aligned workspace, %zu given", name, need, ws_bytes);
  MIQ_REQUIRE(pl.part_bytes == wo_wide_part_bytes(M, N, pl.S), "%s: inconsistent wide plan", name);
  WideParams p{};
  p.x = static_cast<const uint16_t*>(ws);
  p.w = w;
  p.ldw = ldw;
  p.scale = scale;
  p.zero = zero;
  p.group_steps = group_steps;
  p.ngroups = ngroups;
  p.y = y;
  p.ldy = ldy;
  p.M = (int)M;
  p.N = N;
  p.steps = K / kStepK;
  p.tiles_m = (int)((M + 128 * mt - 1) / (128 * mt));
  p.tiles_n = (N + kWN - 1) / kWN;
  p.xbytes = (int)pl.pack_bytes;
  p.wbytes = (int)((int64_t)N * ldw);
  const int esz = sd == MIQ_F32 ? 4 : 2;
  p.sbytes = kind == KIND_INT4 ? (int)(((int64_t)N * ngroups * esz + 3) & ~3LL) : 0;
  p.vec_store = (reinterpret_cast<uintptr_t>(y) & 7) == 0 && ldy % 4 == 0;
  // every XCD reads all of the operand its tiles do not share: keep the larger one shared
  // (each XCD then reads all of the smaller one)
  p.m_major = (int64_t)pl.pack_bytes > (int64_t)N * ldw;
  p.S = pl.S;
  p.split_steps = pl.S > 1 ? pl.split_steps : p.steps;
  p.part = pl.S > 1 ? reinterpret_cast<float*>(static_cast<char*>(ws) + pl.pack_bytes) : nullptr;
  p.split_stride = (M * N + 3) & ~3LL;
  MIQ_REQUIRE((int64_t)p.tiles_m * p.tiles_n * p.S < (1LL << 30), "%s: too many tiles", name);
  const int tiles32 = p.tiles_m * 4 * mt;
  hipLaunchKernelGGL(wo_wide_pack_kernel, dim3(p.steps, tiles32), dim3(256), 0, st, x, ldx, (int)M, p.steps,
                     static_cast<uint16_t*>(ws));
#define MIQ_WIDE_MT(K_, HZ_, SD_)                                   \
  do {                                                              \
    if (mt == 1) launch_wide<K_, HZ_, SD_, 1>(p, st);               \
    else if (mt == 2) launch_wide<K_, HZ_, SD_, 2>(p, st);          \
    else launch_wide<K_, HZ_, SD_, 3>(p, st);                       \
  } while (0)
#define MIQ_WIDE(K_, HZ_)                                           \
  do {                                                              \
    if (sd == MIQ_BF16) MIQ_WIDE_MT(K_, HZ_, MIQ_BF16);             \
    else if (sd == MIQ_F16) MIQ_WIDE_MT(K_, HZ_, MIQ_F16);          \
    else MIQ_WIDE_MT(K_, HZ_, MIQ_F32);                             \
  } while (0)
  if (kind == KIND_INT8) MIQ_WIDE(KIND_INT8, false);
  else if (zero) MIQ_WIDE(KIND_INT4, true);
  else MIQ_WIDE(KIND_INT4, false);
#undef MIQ_WIDE
#undef MIQ_WIDE_MT
  // clear the packed activations again (with K splits, in the reduce kernel's launch)
  const int64_t n16 = (int64_t)(pl.pack_bytes / 16);
  const unsigned clear_blocks = (unsigned)((n16 + 1023) / 1024);
  if (pl.S > 1) {
    const unsigned blocks = clear_blocks + (unsigned)((M * N + 1023) / 1024);
#define MIQ_WIDE_RED(I8_, SD_)                                                                                  \
  hipLaunchKernelGGL((wo_wide_reduce_kernel<I8_, SD_>), dim3(blocks), dim3(256), 0, st, p.part, p.split_stride, \
                     p.S, p.M, p.N, scale, y, ldy, static_cast<i32x4*>(ws), n16, (int)clear_blocks)
    if (kind != KIND_INT8) MIQ_WIDE_RED(false, MIQ_F32);
    else if (sd == MIQ_BF16) MIQ_WIDE_RED(true, MIQ_BF16);
    else if (sd == MIQ_F16) MIQ_WIDE_RED(true, MIQ_F16);
    else MIQ_WIDE_RED(true, MIQ_F32);
#undef MIQ_WIDE_RED
  } else {
    hipLaunchKernelGGL(wo_wide_clear_kernel, dim3(clear_blocks), dim3(256), 0, st, static_cast<i32x4*>(ws), n16);
  }
  return check_launch(name);
}

}  // namespace miq
