// Weight-only quantized GEMM for prefill (M > 64 activation rows), gfx950:
//
//   y[m, n] = sum_k x[m, k] * W[n, k],  x bf16 [M, K],  W int8 [N, K] or int4 [N, K/2]
//
// The weights are dequantized inside the K loop; no bf16 copy of W is ever written.
//
// A workgroup of 4 wavefronts owns a 64 x 128 output tile (64 activation rows x 128
// weight rows); wavefront w owns weight rows 32 w .. 32 w + 31 (two 16-row tiles) over all
// 64 activation rows (four 16-row tiles), so each unpacked weight fragment feeds four
// MFMAs and no weight is unpacked twice in a workgroup. (128 activation rows spill at the
// 256 registers two wavefronts per SIMD leave.)
//   * activations: one k-step (128 k) of the 64 rows at a time goes global -> registers ->
//     LDS (int4: in the nibble-unpack order), double buffered; int4 requests step s + 1 and
//     int8 step s + 2 (two register sets) while step s is multiplied. While a thread writes
//     its pieces it adds
//     them, and a 16-lane DPP reduction gives each row's sum over the step, which removes the
//     +128 code offset;
//   * weights: a unit of 128 bytes per row (two int4 k-steps, one int8 k-step) is loaded as
//     two 16-byte loads per lane and tile in address order (whole 128-byte lines), one unit
//     ahead (int4) or four (int8) in further register sets; lanes_to_mfma turns them into the
//     MFMA B layout (on MI355X the deeper int8 pipeline took 4-9 % off the 2560 x 9728 shape;
//     for int4 it measured 3-5 % slower at 19456 x 2560);
//   * math: v_mfma_f32_16x16x32_bf16 on bf16 128 + code. int4: per k-step
//     acc += s_g * (sum x (128 + u) + bias * sum x) [+ z_g * sum x], with the scale (and
//     zero) of that step's group, so any group size multiple of 128 works; int8: the sums
//     over all K, then y = bf16(bf16(acc - 128 sum x) * bf16(s)) as int8_wo.linear.
// A launch may split K (plan_prefill: so that the items fill whole rounds of resident
// workgroups); the last workgroup of a tile to arrive adds the fp32 partials in split
// order and leaves the workspace zero again.
// Tiles are handed to XCDs in contiguous blocks (consecutive workgroup ids go to different
// XCDs), so an XCD's L2 keeps the weight panels of its block while the activations come
// from the MALL.
#include <algorithm>
#include <type_traits>
#include <utility>

#include "miq_common.h"
#include "wo_core.h"
#include "wo_wide.h"

namespace miq {
namespace {

using namespace wo;

constexpr int kPM = 64, kPN = 128;         // output tile
constexpr int kPieces = kPM * 16 / 256;    // 16-byte activation pieces per thread and k-step
constexpr int kPRow = kStepK + 8;          // LDS row pitch of the staged activations (bf16)

struct PrefillParams {
  const uint16_t* x;
  int64_t ldx;
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
  int wbytes, sbytes;
  int S, split_steps;   // K splits and k-steps per split (a multiple of the unit's steps)
  float* part;          // S > 1: [S][M][N] fp32 partials, zero between calls
  int* counters;        // S > 1: one arrival counter per tile, zero between calls
};

// f(integral_constant<int, 0>) ... f(integral_constant<int, N - 1>), in order
template <int N, int I = 0, class F>
__device__ inline void unroll_n(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    unroll_n<N, I + 1>(f);
  }
}

template <int KIND, bool HZ, int SD>
__global__ void __launch_bounds__(256, 2)
wo_prefill_kernel(PrefillParams p) {
  constexpr bool I4 = KIND == KIND_INT4;
  constexpr int MT = kPM / 16, NT = 2, SPU = I4 ? 2 : 1;  // k-steps per 128-byte unit
  constexpr float kXBias = I4 && !HZ ? -136.f : -128.f;
  __shared__ __align__(16) uint16_t s_x[2][kPM * kPRow];
  __shared__ float s_sum[2][kPM];
  const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, g = lane >> 4;

  // item (K split, tile) of this workgroup: XCD x (= id % 8) takes items
  // [x I / 8, (x + 1) I / 8), split by split, weight panel by weight panel, all activation
  // tiles of a panel in a row (they read the same weight lines)
  const int T = p.tiles_m * p.tiles_n, I = T * p.S;
  const int xcd = blockIdx.x & 7, local = blockIdx.x >> 3;
  const int item = (int)((int64_t)I * xcd / 8) + local;
  if (item >= (int)((int64_t)I * (xcd + 1) / 8)) return;
  const int split = item / T, tile = item - split * T;
  const int tn = tile / p.tiles_m, tm = tile - tn * p.tiles_m;
  const int sb = split * p.split_steps;             // first k-step of the split
  const int ns = min(p.steps - sb, p.split_steps);  // k-steps of the split
  const int m0 = tm * kPM, n0 = tn * kPN + wv * 32;

  // ---- activation staging: piece i = tid + 256 j, row i / 16, 16-byte column i % 16
  int xoff[kPieces];  // element offsets of the thread's pieces (rows past M re-read row M - 1)
#pragma unroll
  for (int j = 0; j < kPieces; ++j) xoff[j] = min(m0 + ((tid + 256 * j) >> 4), p.M - 1) * (int)p.ldx + (tid & 15) * 8;
  // two register sets: the pieces of step s + 2 are requested while step s is multiplied
  uint4 xr[2][kPieces];
  auto stage_load = [&](auto xi_c, int s) {
    constexpr int xi = decltype(xi_c)::value;
#pragma unroll
    for (int j = 0; j < kPieces; ++j)
      xr[xi][j] = *reinterpret_cast<const uint4*>(p.x + xoff[j] + (int64_t)(sb + s) * kStepK);
  };
  auto stage_store = [&](auto xi_c, int buf) {
    constexpr int xi = decltype(xi_c)::value;
#pragma unroll
    for (int j = 0; j < kPieces; ++j) {
      const int row = (tid + 256 * j) >> 4;
      *reinterpret_cast<uint4*>(&s_x[buf][row * kPRow + (tid & 15) * 8]) = I4 ? permute_for_u4(xr[xi][j]) : xr[xi][j];
      float sm = sum8_bf16(xr[xi][j]);
      sm += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sm), 0x111, 0xf, 0xf, true));
      sm += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sm), 0x112, 0xf, 0xf, true));
      sm += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sm), 0x114, 0xf, 0xf, true));
      sm += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sm), 0x118, 0xf, 0xf, true));
      if ((tid & 15) == 15) s_sum[buf][row] = sm * kXBias;
    }
  };

  // ---- weights: load h of a unit covers rows 8h .. 8h + 7 of a tile, 128 bytes each, in
  // address order within each 64-byte half (lane 32 c2 + 4 rr + cl: row 8h + rr, bytes
  // 64 c2 + 16 cl)
  const int lrr = (lane >> 2) & 7, lcl = lane & 3, lc2 = lane >> 5;
  const int bp_addr = (32 * (r >> 3) + 4 * (r & 7) + g) * 4;
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(p.w), 0, p.wbytes, 0x00020000);
  constexpr int kOut = 0x7ffffff0;  // outside every buffer: the load returns zeros
  int wbase[NT][2];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int row = n0 + t * 16 + 8 * h + lrr;
      wbase[t][h] = row < p.N ? row * (int)p.ldw + sb / SPU * 128 + lc2 * 64 + lcl * 16 : -1;
    }
  const int units = (ns + SPU - 1) / SPU;
  // weight units in flight: unit u + WR is requested once unit u has been multiplied
  constexpr int WR = I4 ? 2 : 4;  // INT4: the loop below keeps one unit ahead
  uint4 wb[WR][NT][2];
  // int4: the raw scale / zero words of the unit's k-steps (group of each step)
  const __amdgpu_buffer_rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p.scale), 0, p.sbytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t zrs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(HZ ? p.zero : p.scale), 0, p.sbytes, 0x00020000);
  constexpr int esz = SD == MIQ_F32 ? 4 : 2;
  uint32_t sq[WR][SPU][NT], zq[WR][SPU][NT];
  int srow[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) srow[t] = min(n0 + t * 16 + r, p.N - 1);
  auto load_unit = [&](auto bi_c, int u) {
    constexpr int bi = decltype(bi_c)::value;
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int off = (u < units && wbase[t][h] >= 0) ? wbase[t][h] + u * 128 : kOut;
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(wrs, off, 0, 0);
        wb[bi][t][h] = *reinterpret_cast<const uint4*>(&v);
      }
    if constexpr (I4) {
#pragma unroll
      for (int k = 0; k < SPU; ++k)
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const int s = sb + min(u * SPU + k, ns - 1);
          const int gi = (int)(srow[t] * p.ngroups + s / p.group_steps);
          sq[bi][k][t] = __builtin_amdgcn_raw_buffer_load_b32(srs, (gi * esz) & ~3, 0, 0);
          zq[bi][k][t] = HZ ? __builtin_amdgcn_raw_buffer_load_b32(zrs, (gi * esz) & ~3, 0, 0) : 0u;
        }
    }
  };

  const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
  f32x4 acc[NT][MT], xsg[MT];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[t][mt] = z4;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) xsg[mt] = z4;
  uint4 fr[NT][2];  // the current unit in the MFMA layout

  // multiply k-step k of unit buffer bi from activation buffer buf
  auto compute_step = [&](auto bi_c, auto k_c, int buf, int s) {
    constexpr int bi = decltype(bi_c)::value, k = decltype(k_c)::value;
    if (k == 0) {
#pragma unroll
      for (int t = 0; t < NT; ++t) lanes_to_mfma(bp_addr, wb[bi][t][0], wb[bi][t][1], fr[t][0], fr[t][1]);
    }
    bf16x8 bv[NT][4];
    float sc[NT], zs[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if constexpr (I4) {
        unpack_b<KIND_INT4>(&fr[t][k], bv[t]);
        const int gi = (int)(srow[t] * p.ngroups + (sb + s) / p.group_steps);
        sc[t] = word_to_f32<SD>(sq[bi][k][t], gi);
        zs[t] = HZ ? word_to_f32<SD>(zq[bi][k][t], gi) * (1.f / kXBias) : 0.f;
      } else {
        unpack_b<KIND_INT8>(fr[t], bv[t]);
      }
    }
    const uint16_t* xs = s_x[buf];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const uint16_t* row = xs + (mt * 16 + r) * kPRow;
      bf16x8 av[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint4 v = *reinterpret_cast<const uint4*>(row + a_off<KIND>(0, g, j));
        av[j] = as_bf16x8(v.x, v.y, v.z, v.w);
      }
      const f32x4 xb = *reinterpret_cast<const f32x4*>(&s_sum[buf][mt * 16 + g * 4]);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        if constexpr (I4) {
          f32x4 c = mfma(av[0], bv[t][0], xb);
#pragma unroll
          for (int j = 1; j < 4; ++j) c = mfma(av[j], bv[t][j], c);
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            acc[t][mt][v] = __builtin_fmaf(sc[t], c[v], acc[t][mt][v]);
            if (HZ) acc[t][mt][v] = __builtin_fmaf(zs[t], xb[v], acc[t][mt][v]);
          }
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[t][mt] = mfma(av[j], bv[t][j], acc[t][mt]);
        }
      }
      if constexpr (!I4) xsg[mt] += xb;
    }
  };

  if constexpr (I4) {
    // INT4 (measured faster this way on MI355X than the deeper pipeline below): step s + 1
    // is requested while step s is multiplied and staged right after it; unit u + 1 is
    // requested when unit u starts
    constexpr auto X0 = std::integral_constant<int, 0>{};
    stage_load(X0, 0);
    load_unit(std::integral_constant<int, 0>{}, 0);
    stage_store(X0, 0);
    __syncthreads();
    for (int u = 0; u < units; u += 2) {
      load_unit(std::integral_constant<int, 1>{}, u + 1);
#pragma unroll
      for (int k = 0; k < SPU; ++k) {
        const int s = u * SPU + k;
        if (s < ns) {
          if (s + 1 < ns) stage_load(X0, s + 1);
          if (k == 0) compute_step(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{}, s & 1, s);
          else compute_step(std::integral_constant<int, 0>{}, std::integral_constant<int, SPU - 1>{}, s & 1, s);
          if (s + 1 < ns) stage_store(X0, (s + 1) & 1);
          __syncthreads();
        }
      }
      if (u + 1 >= units) break;
      load_unit(std::integral_constant<int, 0>{}, u + 2);
#pragma unroll
      for (int k = 0; k < SPU; ++k) {
        const int s = (u + 1) * SPU + k;
        if (s < ns) {
          if (s + 1 < ns) stage_load(X0, s + 1);
          if (k == 0) compute_step(std::integral_constant<int, 1>{}, std::integral_constant<int, 0>{}, s & 1, s);
          else compute_step(std::integral_constant<int, 1>{}, std::integral_constant<int, SPU - 1>{}, s & 1, s);
          if (s + 1 < ns) stage_store(X0, (s + 1) & 1);
          __syncthreads();
        }
      }
    }
  } else {
  // ---- prologue: units 0 .. WR - 1 and steps 0, 1 requested, step 0 staged
#pragma unroll
    for (int w = 0; w < WR; ++w) {
      if (w == 0) load_unit(std::integral_constant<int, 0>{}, 0);
      else if (w == 1) load_unit(std::integral_constant<int, 1 % WR>{}, 1);
      else if (w == 2) load_unit(std::integral_constant<int, 2 % WR>{}, 2);
      else load_unit(std::integral_constant<int, 3 % WR>{}, 3);
    }
    stage_load(std::integral_constant<int, 0>{}, 0);
    if (ns > 1) stage_load(std::integral_constant<int, 1>{}, 1);
    stage_store(std::integral_constant<int, 0>{}, 0);
    __syncthreads();
    // ---- main loop: WR units (an even number of steps) per trip, so every register set and
    // LDS buffer index is a compile-time constant. Step s multiplies LDS buffer s & 1,
    // requests step s + 2 into the register set step s came from, stages step s + 1
    // (requested two steps ago) into the other buffer, and after a unit's last step requests
    // unit u + WR into that unit's registers.
    constexpr int kBody = WR * SPU;
    static_assert(kBody % 2 == 0, "steps per trip must be even");
    for (int s0 = 0; s0 < ns; s0 += kBody) {
      unroll_n<kBody>([&](auto i_c) {
        constexpr int i = decltype(i_c)::value, bi = i / SPU, k = i % SPU;
        const int s = s0 + i;
        if (s < ns) {
          if (s + 2 < ns) stage_load(std::integral_constant<int, i & 1>{}, s + 2);
          compute_step(std::integral_constant<int, bi>{}, std::integral_constant<int, k>{}, i & 1, s);
          if (s + 1 < ns) stage_store(std::integral_constant<int, (i + 1) & 1>{}, (i + 1) & 1);
          __syncthreads();
          if (k == SPU - 1) load_unit(std::integral_constant<int, bi>{}, (s0 + i) / SPU + WR);
        }
      });
    }
  }

  // ---- epilogue: lane (r, g) holds y[m0 + 16 mt + 4 g + v][n0 + 16 t + r]
  if (p.S == 1) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int n = n0 + t * 16 + r;
      if (n >= p.N) continue;
      float rs = 1.f;
      if constexpr (!I4) rs = bf16_to_f32(f32_to_bf16(sd_to_f32<SD>(load_sd_raw<SD>(p.scale, n))));
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int m = m0 + mt * 16 + g * 4 + v;
          if (m >= p.M) continue;
          float o = acc[t][mt][v];
          if constexpr (!I4) o = bf16_to_f32(f32_to_bf16(o + xsg[mt][v])) * rs;
          p.y[(int64_t)m * p.ldy + n] = f32_to_bf16(o);
        }
    }
    return;
  }

  // ---- split K: publish the fp32 partial tile with agent-coherent stores, wait for them,
  // then count arrivals; the last workgroup of the tile adds the S partials in split order
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int n = n0 + t * 16 + r;
    if (n >= p.N) continue;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int m = m0 + mt * 16 + g * 4 + v;
        if (m >= p.M) continue;
        const float o = I4 ? acc[t][mt][v] : acc[t][mt][v] + xsg[mt][v];
        __hip_atomic_store(p.part + ((int64_t)split * p.M + m) * p.N + n, o, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's partial stores are done
  __syncthreads();
  __shared__ int s_last;
  if (tid == 0)
    s_last = __hip_atomic_fetch_add(p.counters + tile, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == p.S - 1;
  __syncthreads();
  if (!s_last) return;
  // 4 consecutive outputs per vector; a thread takes vectors tid + 256 j (j < 8) of the
  // 64 x 128 tile, two at a time, requesting 4 splits of each per round with sc1 loads
  // (requests past the last split or outside the output go to an offset outside the buffer:
  // zeros, no memory access), then stores zeros back, so the workspace is all zeros again
  const __amdgpu_buffer_rsrc_t prs =
      __builtin_amdgcn_make_buffer_rsrc(p.part, 0, (int)((int64_t)p.S * p.M * p.N * 4), 0x00020000);
  const int sstride = p.M * p.N * 4, nb = tn * kPN;
  const i32x4 zero4 = {0, 0, 0, 0};
  for (int j0 = 0; j0 < 8; j0 += 2) {
    float4 o[2];
    int off[2];
    bool ok[2];
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int vi = tid + 256 * (j0 + jj);
      const int m = m0 + (vi >> 5), n = nb + (vi & 31) * 4;
      ok[jj] = m < p.M && n < p.N;
      off[jj] = ok[jj] ? (m * p.N + n) * 4 : 0;
      o[jj] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    for (int s0 = 0; s0 < p.S; s0 += 4) {
      float4 t4[4][2];
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
          const int so = ok[jj] && s0 + u < p.S ? off[jj] + (s0 + u) * sstride : kOut;
          const auto w = __builtin_amdgcn_raw_buffer_load_b128(prs, so, 0, 16 /* sc1 */);
          t4[u][jj] = *reinterpret_cast<const float4*>(&w);
        }
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int jj = 0; jj < 2; ++jj)
          if (ok[jj] && s0 + u < p.S)
            __builtin_amdgcn_raw_buffer_store_b128(zero4, prs, off[jj] + (s0 + u) * sstride, 0, 16 /* sc1 */);
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
          o[jj].x += t4[u][jj].x;
          o[jj].y += t4[u][jj].y;
          o[jj].z += t4[u][jj].z;
          o[jj].w += t4[u][jj].w;
        }
    }
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      if (!ok[jj]) continue;
      const int vi = tid + 256 * (j0 + jj);
      const int m = m0 + (vi >> 5), n = nb + (vi & 31) * 4;
      const float f[4] = {o[jj].x, o[jj].y, o[jj].z, o[jj].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float val = f[e];
        if constexpr (!I4)
          val = bf16_to_f32(f32_to_bf16(val)) * bf16_to_f32(f32_to_bf16(sd_to_f32<SD>(load_sd_raw<SD>(p.scale, n + e))));
        p.y[(int64_t)m * p.ldy + n + e] = f32_to_bf16(val);
      }
    }
  }
  if (tid == 0) __hip_atomic_store(p.counters + tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int KIND, bool HZ, int SD>
void launch_prefill(const PrefillParams& p, hipStream_t st) {
  const unsigned items = (unsigned)(p.tiles_m * p.tiles_n * p.S);
  const unsigned grid = (items + 7) / 8 * 8 + 8;  // every XCD block fits its share
  hipLaunchKernelGGL((wo_prefill_kernel<KIND, HZ, SD>), dim3(grid), dim3(256), 0, st, p);
}

struct PrefillPlan {
  int S, split_steps;
  size_t partial_bytes;  // S > 1: [S][M][N] fp32
};

// K splits (whole 128-byte weight units) are chosen by a cost model of the launch. 512
// workgroups are resident at once (2 per CU, 256 CUs), so `tiles * S` items take
// ceil(tiles * S / 512) rounds of steps / S k-steps each; every split adds an fp32 partial
// tile that is stored, counted and read back by the last arriver. On MI355X (INT4 and
// INT8, N x K = 2560 x 9728 and 19456 x 2560, M = 256 ... 2048) the launch time followed
//   rounds * steps * 1.45 us / S  +  (S > 1) * S * M * N * 4 bytes / (1 TB/s)
// to about 10 %: e.g. 2560 x 9728 at M = 512 (160 tiles) took 85 us with S = 4 (640 items,
// two rounds) and 54.5 us with S = 3 (480 items, one round). The S of least modelled time
// is taken (the smaller on ties), with splits of at least 4 k-steps, at most 16 splits,
// partials within kPrefillMaxPartials (so that the no-allocation entry point, whose
// scratch holds that much, plans the same splits) and one counter per tile.
constexpr size_t kPrefillMaxPartials = (size_t)30 << 20;
PrefillPlan plan_prefill(int kind, int64_t M, int64_t N, int64_t K, size_t counter_bytes) {
  const int spu = kind == KIND_INT4 ? 2 : 1;
  const int steps = (int)(K / kStepK);
  const int64_t tiles = ((M + kPM - 1) / kPM) * ((N + kPN - 1) / kPN);
  PrefillPlan pl{1, steps, 0};
  constexpr int64_t kSlots = 2 * 256;  // resident workgroups (2 per CU, 256 CUs)
  constexpr double kStepUs = 1.45, kPartialBytesPerUs = 1e6;
  auto partial_bytes = [&](int S) { return (size_t)S * (size_t)M * (size_t)N * 4; };
  // splits of `per` k-steps (rounded to whole units); returns the split count
  auto splits_for = [&](int S) {
    int per = (steps + S - 1) / S;
    per = (per + spu - 1) / spu * spu;
    return std::pair<int, int>((steps + per - 1) / per, per);
  };
  const bool counters_ok = tiles * 4 <= (int64_t)counter_bytes;
  const int forced = tuning().wo_prefill_s;  // MIQ_WO_PREFILL_S, for tuning runs
  int best_s = 1, best_per = steps;
  if (forced > 0) {
    const auto sp = splits_for(std::min(forced, steps));
    best_s = sp.first;
    best_per = sp.second;
  } else if (counters_ok) {
    double best = (double)((tiles + kSlots - 1) / kSlots) * steps * kStepUs;
    for (int S = 2; S <= 16; ++S) {
      const auto sp = splits_for(S);
      if (sp.first != S || sp.second < 4 || partial_bytes(S) > kPrefillMaxPartials) continue;
      const double cost = (double)((tiles * S + kSlots - 1) / kSlots) * steps * kStepUs / S +
                          (double)partial_bytes(S) / kPartialBytesPerUs;
      if (cost < best) {
        best = cost;
        best_s = S;
        best_per = sp.second;
      }
    }
  }
  if (best_s <= 1) return pl;
  pl.S = best_s;
  pl.split_steps = best_per;
  pl.partial_bytes = partial_bytes(best_s);
  return pl;
}

}  // namespace

// Plan of the wide kernel for this call (mt = 0: the prefill kernel): M from MIQ_WO_WIDE_MIN_M
// up, the wide kernel not switched off.
static WidePlan wide_plan(int64_t M, int64_t N, int64_t K, int64_t ldw) {
  if (tuning().wo_wide_mt == 0 || M < tuning().wo_wide_min_m) return WidePlan{};
  return wo_wide_plan(M, N, K, ldw);
}

// Workspace bytes of a prefill call: the counter area, then the split-K partials or (with_wide)
// the wide kernel's packed activations, whichever is larger.
size_t wo_prefill_workspace_bytes(int64_t M, int64_t N, int64_t K, int weight_bits, size_t counter_bytes,
                                  bool with_wide) {
  const PrefillPlan pl = plan_prefill(weight_bits == 4 ? KIND_INT4 : KIND_INT8, M, N, K, counter_bytes);
  const size_t split = pl.S > 1 ? counter_bytes + pl.partial_bytes : 0;
  // the wide kernel's packed activations and partials (ldw is not known here: its limit is
  // checked at launch)
  const WidePlan wp = with_wide ? wide_plan(M, N, K, 0) : WidePlan{};
  const size_t wide = wp.mt > 0 ? counter_bytes + wp.bytes() : 0;
  return std::max(split, wide);
}

// Launches the prefill kernel (any M >= 1; meant for M > 64); returns a MIQ_* status. With a
// K split, the per-tile arrival counters are the first ints of the workspace and the
// partials start at byte `counter_bytes`; both are zero between calls and left zero.
int wo_prefill_launch(int kind, const uint16_t* x, int64_t ldx, const uint8_t* w, int64_t ldw, const void* scale,
                      const void* zero, int sd, int group_steps, int64_t ngroups, uint16_t* y, int64_t ldy, int64_t M,
                      int N, int K, void* workspace, size_t ws_bytes, size_t counter_bytes, hipStream_t st,
                      const char* name) {
  // the wide kernel where it is planned and its workspace fits (the no-allocation entry
  // point's scratch may not hold it: then the prefill kernel)
  if (workspace != nullptr && ws_bytes > counter_bytes) {
    const WidePlan wp = wide_plan(M, N, K, ldw);
    if (wp.mt > 0 && ws_bytes - counter_bytes >= wp.bytes())
      return wo_wide_launch(kind, wp, x, ldx, w, ldw, scale, zero, sd, group_steps, ngroups, y, ldy, M, N, K,
                            static_cast<char*>(workspace) + counter_bytes,
                            ws_bytes - counter_bytes, st, name);
  }
  MIQ_REQUIRE((int64_t)N * ldw < 0x7fff0000LL, "%s: weights of %lld bytes exceed 2 GiB", name, (long long)N * ldw);
  MIQ_REQUIRE(M * ldx < (1LL << 31), "%s: activations of %lld elements exceed 2^31", name, (long long)(M * ldx));
  const PrefillPlan pl = plan_prefill(kind, M, N, K, counter_bytes);
  PrefillParams p{};
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
  p.M = (int)M;
  p.N = N;
  p.steps = K / kStepK;
  p.tiles_m = (int)((M + kPM - 1) / kPM);
  p.tiles_n = (N + kPN - 1) / kPN;
  p.wbytes = (int)((int64_t)N * ldw);
  const int esz = sd == MIQ_F32 ? 4 : 2;
  p.sbytes = kind == KIND_INT4 ? (int)(((int64_t)N * ngroups * esz + 3) & ~3LL) : 0;
  p.S = pl.S;
  p.split_steps = pl.split_steps;
  MIQ_REQUIRE((int64_t)p.tiles_m * p.tiles_n * p.S < (1LL << 30), "%s: too many tiles", name);
  if (pl.S > 1) {
    MIQ_REQUIRE(pl.partial_bytes < (1u << 31) && (int64_t)p.tiles_m * p.tiles_n * 4 <= (int64_t)counter_bytes,
                "%s: split-K plan out of range", name);
    MIQ_REQUIRE(workspace != nullptr && ws_bytes >= counter_bytes + pl.partial_bytes,
                "%s: workspace of %zu bytes is below the %zu this call needs", name, ws_bytes,
                counter_bytes + pl.partial_bytes);
    p.counters = static_cast<int*>(workspace);
    p.part = reinterpret_cast<float*>(static_cast<char*>(workspace) + counter_bytes);
  }
#define MIQ_PREFILL(K_, HZ_)                                                         \
  do {                                                                               \
    if (sd == MIQ_BF16) launch_prefill<K_, HZ_, MIQ_BF16>(p, st);                    \
    else if (sd == MIQ_F16) launch_prefill<K_, HZ_, MIQ_F16>(p, st);                 \
    else launch_prefill<K_, HZ_, MIQ_F32>(p, st);                                    \
  } while (0)
  if (kind == KIND_INT8) MIQ_PREFILL(KIND_INT8, false);
  else if (zero) MIQ_PREFILL(KIND_INT4, true);
  else MIQ_PREFILL(KIND_INT4, false);
#undef MIQ_PREFILL
  return check_launch(name);
}

}  // namespace miq
