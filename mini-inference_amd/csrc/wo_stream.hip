// Weight-only quantized skinny GEMM (1 <= M <= 64) for gfx950:
//
//   y[m, n] = sum_k x[m, k] * W[n, k],  x bf16 [M, K],  W int8 [N, K] or int4 [N, K/2]
//
// Work decomposition:
//   * a workgroup of W wavefronts (4 for one activation tile, 8 for several) owns a row
//     block of W * NR tiles of 16 weight rows and a K range (one of S splits along
//     grid.y); wavefront w owns tiles w * NR .. + NR - 1 over the whole range, so the
//     activations it multiplies are shared by the W wavefronts through LDS (x is read
//     from L2 once per row block, not once per tile);
//   * the activations of a chunk of the range are staged in LDS by a short loop; while a
//     thread writes its pieces it also adds their 8 values, and a 16-lane DPP reduction
//     gives sum_k x over every k-step, which removes the +128 code offset (below) with 4
//     FMAs per group instead of one MFMA per operand;
//   * weights stream through a ring of D k-steps of registers: step k + D is requested
//     (16-byte buffer loads, one per lane; non-temporal except in the M split) right
//     after step k has been multiplied, so D steps are always in flight and the wait
//     before a step is a constant count. Requests past the range use an offset outside
//     the buffer, which the hardware answers with zeros without touching memory;
//   * M split (int4, M > 16): grid.z runs over the 16-row activation tiles, each
//     workgroup taking one of them with two weight tiles per wavefront; the workgroups of
//     one row block on different activation tiles read the same weight lines (same XCD);
//   * the code is a pair of short loops: these kernels run for a few microseconds, and
//     the instruction fetch of straight-line code costs about as much as the loads;
//   * with S > 1 every workgroup publishes fp32 partials with agent-coherent (sc1)
//     stores, waits for them and bumps a per-row-block arrival counter; the last one adds
//     the S partials in split order (deterministic), writes bf16, sets the partials it
//     read back to zero and resets the counter, so the workspace is all zeros between calls.
//
// Unpacking: a 4-bit code u becomes the bf16 value 128 + u with one AND-OR per pair
// (0x4300 | u == 128 + u, exact) and an int8 code q becomes 128 + q via xor + byte
// convert. The MFMA yields sum x * (128 + u); the staged sums hold bias * sum x (bias
// -136 for symmetric int4 codes u - 8, -128 with zero points and for int8), and per
// group (int4)
//   acc += scale * (sum x (128 + u) + bias * sum x)  [+ zero * sum x with zero points]
// and per row (int8) y = bf16(bf16(sum x (128 + q) - 128 sum x) * bf16(scale)).
// One-step (128-code) int4 groups have their own instantiation (G1): each k-step's
// MFMA chains start from its bias sums and from zero, and end the group at once.
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>
#include <type_traits>

#include <mutex>

#include "wo_core.h"

#ifndef MIQ_TRACE
#define MIQ_TRACE(point)
#endif

// ring depth (k-steps of int4 weights in flight per wavefront, divided by NR) for one
// activation tile; 8 and 16 measured slower on MI355X (their registers cost occupancy)
#ifndef MIQ_D1
#define MIQ_D1 4
#endif

namespace miq {
namespace {

using namespace wo;

// wavefronts per workgroup: 4 for one activation tile (8 and 16 measured slower); 8 for
// several (one weight tile each: twice the wavefronts per SIMD over the same staged
// activations; int8 gate/up on MI355X, M = 32 / 64: 20.4 / 30.5 against 21.6 / 33.5 us
// with 4 wavefronts of two tiles)
template <int MT>
constexpr int waves_for() { return MT >= 2 ? 8 : 4; }
constexpr int kMaxCounters = 4096;   // row blocks that may use split-K
constexpr int kCounterBytes = kMaxCounters * 4;

// ring depth in k-steps (int4 loads come in pairs of k-steps, so at least 2)
constexpr int ring_depth(int kind, int mt, int nr) {
  const int d = (kind == KIND_INT4 ? (mt == 1 ? MIQ_D1 : (mt >= 3 && nr == 1 ? 4 : 8))
                                   : (mt == 1 ? MIQ_D1 / 2 : (mt >= 3 && nr == 1 ? 2 : 4))) / nr;
  return kind == KIND_INT4 ? (d < 2 ? 2 : d) : (d < 1 ? 1 : d);
}

// Compile-time shape of one instantiation: MT tiles of 16 activation rows, NR weight
// tiles per wavefront, D k-steps of weights in flight per wavefront (8 KiB).
template <int KIND, int MT, int NR>
struct Cfg {
  static constexpr int NL = KIND == KIND_INT4 ? 1 : 2;       // 16-byte loads per tile-step
  // ring depth in k-steps: 8 KiB of weights per wavefront (4 KiB for 3-4 activation
  // tiles with one weight tile, so that a chunk of D k-steps of activations fits LDS)
  static constexpr int D = ring_depth(KIND, MT, NR);
  static constexpr int XR = 16 * MT;                          // x-sum row pitch
  static constexpr int XP = 4;                                // staging pieces per thread per round
};

struct StreamParams {
  const uint16_t* x;
  int64_t ldx;
  const uint8_t* w;
  int64_t ldw;          // bytes per weight row
  const void* scale;
  const void* zero;
  int group_steps;      // int4: k-steps per quantization group (1 for int8)
  int64_t ngroups;      // int4: groups per weight row
  uint16_t* y;
  int64_t ldy;
  int M, N;
  int S, units, unit_steps;
  int chunk_steps;      // k-steps of x staged in LDS at once (a multiple of D)
  int wbytes, sbytes;   // sizes of the weight and scale / zero buffers
  float* partial;       // [S][M][N]
  int* counters;        // [kMaxCounters]
};

template <int KIND, bool HZ, int SD, int MT, int NR, bool G1>
__global__ void __launch_bounds__(waves_for<MT>() * 64)
wo_stream_kernel(StreamParams p_in) {
  // M split (grid.z > 1, one activation tile each): this workgroup's 16 rows of x and y,
  // and its own slices of the partials and counters
  StreamParams p = p_in;
  if (gridDim.z > 1) {
    const int m0 = blockIdx.z * 16;
    p.x += (int64_t)m0 * p.ldx;
    p.y += (int64_t)m0 * p.ldy;
    p.partial += (int64_t)blockIdx.z * p.S * 16 * p.N;
    p.counters += blockIdx.z * gridDim.x;
    p.M = min(16, p.M - m0);
  }
  constexpr int kWaves = waves_for<MT>(), kThreads = kWaves * 64;
  using C = Cfg<KIND, MT, NR>;
  constexpr int D = C::D, NL = C::NL, XR = C::XR, XP = C::XP;
  constexpr int kStepBytes = KIND == KIND_INT4 ? kStepK / 2 : kStepK;  // per weight row
  extern __shared__ __align__(16) uint16_t lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, g = lane >> 4;
  const int M = p.M;
  MIQ_TRACE(0);
#ifdef MIQ_TRACE_ARGS
  asm volatile("" ::"s"(M), "s"(p.w), "s"(p.x));
  MIQ_TRACE(5);
#endif

  // K range of this split, in whole units (k-steps for int8, groups for int4)
  const int s = blockIdx.y;
  const int u0 = (int)((int64_t)p.units * s / p.S), u1 = (int)((int64_t)p.units * (s + 1) / p.S);
  const int st0 = u0 * p.unit_steps, st1 = u1 * p.unit_steps;

  // this wavefront's weight rows (rows past N re-read row N - 1; never stored) and the
  // byte offsets of their k-step st0 in the weight / scale buffers
  const int nblk0 = blockIdx.x * (kWaves * NR * 16);
  // Weight loads read whole 128-byte lines: load h of a tile covers its rows 8h..8h+7, 128
  // bytes each (two int4 k-steps, one int8 k-step), in address order within each 64-byte
  // half: lane 32 c2 + 4 rr + cl reads row 8h + rr, bytes 64 c2 + 16 cl. lanes_to_mfma()
  // turns the two loads into the per-k-step MFMA layout (lane (g, r): row r, chunk g of
  // each 64-byte half).
  int nrow[NR], woff[NR][2], soff[NR];
  const int lrr = (lane >> 2) & 7, lcl = lane & 3, lc2 = lane >> 5;
  const int bp_addr = (32 * (r >> 3) + 4 * (r & 7) + g) * 4;
#pragma unroll
  for (int t = 0; t < NR; ++t) {
    nrow[t] = nblk0 + (wv * NR + t) * 16 + r;
    const int nc = min(nrow[t], p.N - 1);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int nh = min(nblk0 + (wv * NR + t) * 16 + 8 * h + lrr, p.N - 1);
      woff[t][h] = nh * (int)p.ldw + st0 * kStepBytes + lc2 * 64 + lcl * 16;
    }
    soff[t] = (int)(nc * p.ngroups + st0 / p.group_steps);  // element index of the first group
  }
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(p.w), 0, p.wbytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p.scale), 0, p.sbytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t zrs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(HZ ? p.zero : p.scale), 0, p.sbytes, 0x00020000);
  constexpr int kOut = 0x7ffffff0;  // an offset outside every buffer: the load returns zeros

  // ring of D k-steps: weights and (int4) the raw scale / zero word of each step's group
  uint4 wq[D][NR][NL];
  uint32_t sq[D][NR], zq[D][NR];
  // steps in the range, as an opaque per-lane value: requests past it are steered to
  // kOut with bit operations (a select would become a branch around each load, and
  // branches cost the precise waits)
  int nsteps_v = st1 - st0;
  asm volatile("" : "+v"(nsteps_v));
  // quantization group of the next request, and its k-steps still to request (requests
  // come in k order), kept as uniform counters instead of divisions
  int rq_grp = 0, rq_left = p.group_steps;
  // int4: the raw loads of k-steps d and d + 1 (d even) sit in wq[d][t][0] and wq[d + 1][t][0];
  // int8: those of k-step d in wq[d][t][0..1]
  // weight loads are non-temporal, except in the M split (MT == 1 with several weight
  // tiles per wavefront), where the workgroups of the other activation tiles read the same
  // lines from L2 (measured 5 % faster at M = 32 and 64 on MI355X than nt)
  constexpr int kWAux = (MT == 1 && NR >= 2) ? 0 : 2 /* nt */;
  auto request = [&](int d, int kl) {  // k-step st0 + kl into slot d
    const int keep = (kl - nsteps_v) >> 31;  // all ones while kl < steps in range
#pragma unroll
    for (int t = 0; t < NR; ++t) {
      if (KIND == KIND_INT8 || (d & 1) == 0) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          // int4 chunks 4..7 hold k-step kl + 1
          const int kp = KIND == KIND_INT4 ? (kl + lc2 - nsteps_v) >> 31 : keep;
          const int off = ((woff[t][h] + kl * kStepBytes) & kp) | (kOut & ~kp);
          const auto v = __builtin_amdgcn_raw_buffer_load_b128(wrs, off, 0, kWAux);
          if (KIND == KIND_INT4) wq[d + h][t][0] = *reinterpret_cast<const uint4*>(&v);
          else wq[d][t][h] = *reinterpret_cast<const uint4*>(&v);
        }
      }
      if (KIND == KIND_INT4) {
        const int gi = soff[t] + rq_grp;
        constexpr int esz = SD == MIQ_F32 ? 4 : 2;
        const int so = ((gi * esz) & ~3 & keep) | (kOut & ~keep);
        sq[d][t] = __builtin_amdgcn_raw_buffer_load_b32(srs, so, 0, 0);
        zq[d][t] = HZ ? __builtin_amdgcn_raw_buffer_load_b32(zrs, so, 0, 0) : 0u;
      }
    }
    if (--rq_left == 0) {
      ++rq_grp;
      rq_left = p.group_steps;
    }
  };
  static_assert(KIND == KIND_INT8 || D % 2 == 0, "int4 loads come in pairs of k-steps");

  // LDS: x chunk [M rows x (CS * 128 + 8)] bf16, then [CS][XR] fp32 sums per k-step
  const int CS = p.chunk_steps;
  const int xstride = CS * kStepK + 8;
  float* xsum = reinterpret_cast<float*>(lds + M * xstride);
  const int xld = (int)(p.ldx / 8);
  const __amdgpu_buffer_rsrc_t xrs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(p.x), 0, (int)((int64_t)M * p.ldx * 2), 0x00020000);
  // activation pieces (16 bytes) of chunk c0, round `base`: XP per thread; pieces j of a
  // round that no thread needs are not loaded (a uniform branch)
  uint4 xr[XP];
  auto load_x = [&](int c0, int base) {
    const int xcols = min(CS, st1 - c0) * (kStepK / 8);
    const int npieces = M * xcols;
    const uint4* xsrc = reinterpret_cast<const uint4*>(p.x) + (int64_t)c0 * (kStepK / 8);
#pragma unroll
    for (int j = 0; j < XP; ++j) {
      if (base + j * kThreads < npieces) {
        const int i = min(base + tid + j * kThreads, npieces - 1);
        const int m = i / xcols, c = i - m * xcols;
        xr[j] = xsrc[(int64_t)m * xld + c];
      }
    }
  };
  // with one activation tile the first activations are requested ahead of the weights
  // (loads complete in order, so staging them does not wait for the weights); with more
  // tiles that measured slower on MI355X
  if (MT == 1) load_x(st0, 0);
#pragma unroll
  for (int d = 0; d < D; ++d) request(d, d);
  MIQ_TRACE(1);
  uint4 wnext[NR];  // int4: the second k-step of the pair being multiplied

  // two MFMA accumulation chains per tile (even / odd j), so consecutive MFMAs do not
  // wait for each other's results
  // Per quantization group, T = sum_k x (128 + u) + kXBias * sum_k x (two MFMA chains and
  // the staged sums, which hold kXBias times the sum of x over each k-step), and
  // acc += s * T (+ z * sum_k x with zero points)
  constexpr float kXBias = KIND == KIND_INT4 && !HZ ? -136.f : -128.f;
  f32x4 acc[NR][MT], accg[NR][MT], acc2[NR][MT], xsg[MT];
  const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int t = 0; t < NR; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) { acc[t][mt] = z4; accg[t][mt] = z4; acc2[t][mt] = z4; }
  int c_grp = 0, c_left = p.group_steps;  // the multiply loop's group and steps left in it
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) xsg[mt] = z4;

  for (int c0 = st0; c0 < st1; c0 += CS) {
    const int nst = min(CS, st1 - c0);
    const int xcols = nst * (kStepK / 8);  // 16-byte pieces per activation row
    const int npieces = M * xcols;
    if (c0 != st0) __syncthreads();  // every wavefront is done with the previous chunk
    if constexpr (KIND == KIND_INT8 && MT >= 2) {
      // Several activation tiles (int8): the chunk's rows go from memory straight into their LDS
      // rows (buffer_load ... lds, one round trip for the whole chunk: staging through
      // registers took one round trip per 16 KiB), and one LDS pass forms the per-k-step
      // sums. For int4 the register path measured the same (its activations are permuted
      // to the unpack order on the way).
      const int ipr = (xcols + 63) / 64;  // loads of up to 64 pieces per row
      const int nload = M * ipr;
      for (int q = wv; q < nload; q += kWaves) {
        const int m = q / ipr, p0 = (q - m * ipr) * 64;
        if (p0 + lane < xcols)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(
              xrs, (__attribute__((address_space(3))) void*)(lds + m * xstride + p0 * 8), 16,
              (m * (int)p.ldx + c0 * kStepK + (p0 + lane) * 8) * 2, 0, 0, 0);
      }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      for (int i0 = 0; i0 < npieces; i0 += kThreads) {
        const int i = i0 + tid;
        const int ic = min(i, npieces - 1);
        const int m = ic / xcols, c = ic - m * xcols;
        const uint4 v = *reinterpret_cast<const uint4*>(lds + m * xstride + c * 8);
        float sm = sum8_bf16(v);
        sm += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sm), 0x111, 0xf, 0xf, true));
        sm += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sm), 0x112, 0xf, 0xf, true));
        sm += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sm), 0x114, 0xf, 0xf, true));
        sm += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sm), 0x118, 0xf, 0xf, true));
        if (i < npieces && (c & 15) == 15) xsum[(c >> 4) * XR + m] = sm * kXBias;
      }
    }
    for (int base = 0; base < (KIND == KIND_INT8 && MT >= 2 ? 0 : npieces); base += XP * kThreads) {
      if (MT > 1 || c0 != st0 || base != 0) load_x(c0, base);
#pragma unroll
      for (int j = 0; j < XP; ++j) {
        if (base + j * kThreads >= npieces) break;
        const int i = base + tid + j * kThreads;
        const int ic = min(i, npieces - 1);
        const int m = ic / xcols, c = ic - m * xcols;
        *reinterpret_cast<uint4*>(lds + m * xstride + c * 8) = KIND == KIND_INT4 ? permute_for_u4(xr[j]) : xr[j];
        // sum over the 16 pieces of one k-step (16 consecutive lanes, one DPP row):
        // lane 15 of the row ends with the total
        float sm = sum8_bf16(xr[j]);
        sm += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sm), 0x111, 0xf, 0xf, true));
        sm += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sm), 0x112, 0xf, 0xf, true));
        sm += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sm), 0x114, 0xf, 0xf, true));
        sm += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sm), 0x118, 0xf, 0xf, true));
        if (i < npieces && (c & 15) == 15) xsum[(c >> 4) * XR + m] = sm * kXBias;
      }
    }
    __syncthreads();
    if (c0 == st0) MIQ_TRACE(2);

    // multiply the chunk, D k-steps per trip; the ring slot of step kl is kl % D
    for (int k = c0; k < c0 + nst; k += D) {
#pragma unroll
      for (int d = 0; d < D; ++d) {
        const int kst = k + d, kl = kst - c0;
        if (kst < c0 + nst) {
          bf16x8 av[MT][4];
          f32x4 xb[MT];
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            const uint16_t* row = lds + min(mt * 16 + r, M - 1) * xstride;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const uint4 v = *reinterpret_cast<const uint4*>(row + a_off<KIND>(kl, g, j));
              av[mt][j] = as_bf16x8(v.x, v.y, v.z, v.w);
            }
            xb[mt] = *reinterpret_cast<const f32x4*>(xsum + kl * XR + mt * 16 + g * 4);
            if (!G1) xsg[mt] += xb[mt];
          }
#pragma unroll
          for (int t = 0; t < NR; ++t) {
            bf16x8 bv[4];
            uint4 wl[2];
            if (KIND == KIND_INT8) {
              lanes_to_mfma(bp_addr, wq[d][t][0], wq[d][t][1], wl[0], wl[1]);
            } else if ((d & 1) == 0) {
              lanes_to_mfma(bp_addr, wq[d][t][0], wq[d + 1][t][0], wl[0], wnext[t]);
            } else {
              wl[0] = wnext[t];
            }
            unpack_b<KIND>(wl, bv);
            if (G1) {
              // one-step groups: the first chain starts from the step's bias, the second
              // from zero, and the group ends here
              const int gi = soff[t] + c_grp;
              const float sc = word_to_f32<SD>(sq[d][t], gi);
              const float zs = HZ ? word_to_f32<SD>(zq[d][t], gi) * (1.f / kXBias) : 0.f;
#pragma unroll
              for (int mt = 0; mt < MT; ++mt) {
                f32x4 c0v = mfma(av[mt][0], bv[0], xb[mt]);
                f32x4 c1v = mfma(av[mt][1], bv[1], z4);
                c0v = mfma(av[mt][2], bv[2], c0v);
                c1v = mfma(av[mt][3], bv[3], c1v);
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[t][mt][v] = __builtin_fmaf(sc, c0v[v] + c1v[v], acc[t][mt][v]);
                if (HZ) {
#pragma unroll
                  for (int v = 0; v < 4; ++v) acc[t][mt][v] = __builtin_fmaf(zs, xb[mt][v], acc[t][mt][v]);
                }
              }
              continue;
            }
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
              for (int j = 0; j < 4; ++j) {
                f32x4& chain = (j & 1) ? acc2[t][mt] : (KIND == KIND_INT4 ? accg[t][mt] : acc[t][mt]);
                chain = mfma(av[mt][j], bv[j], chain);
              }
          }
          if (G1) {
            ++c_grp;
          } else if (KIND == KIND_INT4 && --c_left == 0) {  // end of a quantization group
#pragma unroll
            for (int t = 0; t < NR; ++t) {
              const int gi = soff[t] + c_grp;
              const float sc = word_to_f32<SD>(sq[d][t], gi);
              const float zs = HZ ? word_to_f32<SD>(zq[d][t], gi) * (1.f / kXBias) : 0.f;
#pragma unroll
              for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[t][mt][v] = __builtin_fmaf(sc, accg[t][mt][v] + acc2[t][mt][v] + xsg[mt][v], acc[t][mt][v]);
                if (HZ) {
#pragma unroll
                  for (int v = 0; v < 4; ++v) acc[t][mt][v] = __builtin_fmaf(zs, xsg[mt][v], acc[t][mt][v]);
                }
                accg[t][mt] = z4;
                acc2[t][mt] = z4;
              }
            }
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) xsg[mt] = z4;
            ++c_grp;
            c_left = p.group_steps;
          }
        }
        request(d, kst + D - st0);
      }
    }
  }
  if (KIND == KIND_INT8) {
#pragma unroll
    for (int t = 0; t < NR; ++t)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[t][mt][v] += acc2[t][mt][v] + xsg[mt][v];
  }

  MIQ_TRACE(3);
  // ---- epilogue: lane (r, g) holds y[16 mt + 4 g + v][nrow[t]]
  const bool split = p.S > 1;
#pragma unroll
  for (int t = 0; t < NR; ++t) {
    const int n = nrow[t];
    if (n >= p.N) continue;
    float rs = 1.f;
    if (KIND == KIND_INT8 && !split) rs = bf16_to_f32(f32_to_bf16(sd_to_f32<SD>(load_sd_raw<SD>(p.scale, n))));
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int m = mt * 16 + g * 4 + v;
        if (m >= M) continue;
        const float o = acc[t][mt][v];
        if (split) {
          __hip_atomic_store(p.partial + ((int64_t)s * M + m) * p.N + n, o, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
          p.y[(int64_t)m * p.ldy + n] = f32_to_bf16(KIND == KIND_INT8 ? bf16_to_f32(f32_to_bf16(o)) * rs : o);
        }
      }
  }
  if (!split) return;

  // ---- split-K: the last workgroup of this row block adds the S partials in order
  // this thread's partial stores have completed (the clobber keeps them above the wait)
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  MIQ_TRACE(4);
  __syncthreads();
  __shared__ int s_last;
  if (tid == 0)
    s_last = __hip_atomic_fetch_add(p.counters + blockIdx.x, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == p.S - 1;
  __syncthreads();
  MIQ_TRACE(6);
  if (!s_last) return;
  // 4 consecutive n per thread and round; the S partials of VB such vectors are
  // requested SU splits at a time (VB * SU = 16 loads in flight) with agent-coherent (sc1)
  // 16-byte loads, then added in split order (a missing split adds zeros). VB is the most
  // vectors a thread can have (at most 4 per round).
  constexpr int kRows = kWaves * NR * 16;
  constexpr int kMaxVec = MT * 16 * (kRows / 4);
  constexpr int VB = (kMaxVec + kThreads - 1) / kThreads < 4 ? (kMaxVec + kThreads - 1) / kThreads : 4;
  constexpr int SU = 16 / VB;
  const __amdgpu_buffer_rsrc_t prs =
      __builtin_amdgcn_make_buffer_rsrc(p.partial, 0, (int)((int64_t)p.S * M * p.N * 4), 0x00020000);
  const int nvec = M * (kRows / 4);
  for (int b0 = 0; b0 < nvec; b0 += kThreads * VB) {
    const int v0 = b0 + tid;
    float4 o[VB];
    int off[VB];
    bool ok[VB];
#pragma unroll
    for (int j = 0; j < VB; ++j) {
      const int v = min(v0 + j * kThreads, nvec - 1);
      const int m = v / (kRows / 4), n = nblk0 + (v - m * (kRows / 4)) * 4;
      ok[j] = v0 + j * kThreads < nvec && n < p.N;
      off[j] = (m * p.N + min(n, p.N - 4)) * 4;
      o[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    const int sstride = M * p.N * 4;
    // SU splits per round; 4 when there are at most 4 (fewer requests that go nowhere)
    auto rounds = [&](auto su_c) {
      constexpr int SUR = decltype(su_c)::value;
      for (int s0 = 0; s0 < p.S; s0 += SUR) {
        float4 t[SUR][VB];
        // requests past the last split or vector go to an offset outside the buffer
        // (zeros, no memory access): straight-line code, so the waits stay exact
#pragma unroll
        for (int j = 0; j < VB; ++j)
#pragma unroll
          for (int u = 0; u < SUR; ++u) {
            const bool live = s0 + u < p.S && b0 + j * kThreads < nvec;
            const int so = live ? off[j] + (s0 + u) * sstride : 0x7ffffff0;
            const auto w = __builtin_amdgcn_raw_buffer_load_b128(prs, so, 0, 16 /* sc1 */);
            t[u][j] = *reinterpret_cast<const float4*>(&w);
          }
        // the partials go back to zero once read: the workspace holds zeros between calls
        // (the panel kernel, which shares it, reads a non-zero word as a pending partial)
        const i32x4 zero4 = {0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < VB; ++j)
#pragma unroll
          for (int u = 0; u < SUR; ++u) {
            // only this thread's own vectors (clamped duplicates are read by their owner)
            if (s0 + u < p.S && ok[j]) __builtin_amdgcn_raw_buffer_store_b128(zero4, prs, off[j] + (s0 + u) * sstride, 0, 16 /* sc1 */);
          }
#pragma unroll
        for (int u = 0; u < SUR; ++u)
#pragma unroll
          for (int j = 0; j < VB; ++j) {
            o[j].x += t[u][j].x;
            o[j].y += t[u][j].y;
            o[j].z += t[u][j].z;
            o[j].w += t[u][j].w;
          }
      }
    };
    if (SU > 4 && p.S <= 4) rounds(std::integral_constant<int, 4>{});
    else rounds(std::integral_constant<int, SU>{});
#pragma unroll
    for (int j = 0; j < VB; ++j) {
      if (!ok[j]) continue;
      const int v = v0 + j * kThreads;
      const int m = v / (kRows / 4), n = nblk0 + (v - m * (kRows / 4)) * 4;
      const float f[4] = {o[j].x, o[j].y, o[j].z, o[j].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float val = f[e];
        if (KIND == KIND_INT8)
          val = bf16_to_f32(f32_to_bf16(val)) * bf16_to_f32(f32_to_bf16(sd_to_f32<SD>(load_sd_raw<SD>(p.scale, n + e))));
        p.y[(int64_t)m * p.ldy + n + e] = f32_to_bf16(val);
      }
    }
  }
  if (tid == 0) __hip_atomic_store(p.counters + blockIdx.x, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  MIQ_TRACE(7);
}

// ------------------------------------------------------------------ host-side planning
struct StreamPlan {
  int MT, NR, D, S, units, unit_steps, blocks, chunk_steps;
  int mtiles;  // > 1: the M split (one tile of 16 activation rows per workgroup)
  size_t lds_bytes, partial_bytes;
};

constexpr int kLdsBudget = 80 * 1024;  // two workgroups per CU

StreamPlan plan_stream(int kind, int64_t M, int64_t N, int64_t K, int group_steps) {
  StreamPlan pl{};
  const int64_t steps = K / kStepK;
  pl.unit_steps = kind == KIND_INT4 ? group_steps : 1;
  // int4 splits start on an even k-step when they can, so each weight load covers whole
  // 128-byte lines
  if (kind == KIND_INT4 && group_steps % 2 == 1 && steps % (2 * group_steps) == 0) pl.unit_steps = 2 * group_steps;
  pl.units = (int)(steps / pl.unit_steps);
  pl.MT = (int)((M + 15) / 16);
  pl.mtiles = 1;
  // one weight tile per wavefront: several activation tiles take eight-wavefront
  // workgroups (a row block of 128 rows, as two tiles per wavefront of four did)
  pl.NR = 1;
  int S = 0;
  // M split: one activation tile of 16 rows per workgroup and two weight tiles per
  // wavefront. The workgroups of one row block on its different activation tiles share
  // the weights through L2, and each re-reads 16 activation rows instead of all M. For
  // int4 this measured up to 12 % faster on MI355X (int8 slower), best with about 480
  // workgroups. MIQ_WO_MSPLIT="NR,S" (NR 2 or 4) forces a plan, for tuning; "0,0" off.
  const Tuning& tu = tuning();
  int m_nr = tu.wo_msplit_nr, m_s = tu.wo_msplit_s;
  const bool m_env = tu.wo_msplit_set;
  if (!m_env && kind == KIND_INT4 && M > 16) {
    m_nr = 2;
    const int64_t blocks2 = (N + 127) / 128, tiles = (M + 15) / 16;
    m_s = (int)std::max<int64_t>(1, (480 + blocks2 * tiles / 2) / (blocks2 * tiles));
  }
  if (M > 16 && (m_nr == 2 || m_nr == 4) && m_s >= 1) {
    pl.mtiles = pl.MT;
    pl.MT = 1;
    pl.NR = m_nr;
    S = m_s;
    M = 16;  // per workgroup
  }
  const bool env = pl.mtiles == 1 && tu.wo_plan_set;  // "NR,S" override for tuning
  const int e_nr = tu.wo_plan_nr, e_s = tu.wo_plan_s;
  if (env && (e_nr == 1 || e_nr == 2) && e_s >= 1) {
    if (pl.MT >= 2 || e_nr == 1) pl.NR = e_nr;
    S = e_s;
  }
  pl.D = ring_depth(kind, pl.MT, pl.NR);  // Cfg<>::D
  const int64_t rows = (pl.MT == 1 ? waves_for<1>() : waves_for<2>()) * pl.NR * 16;
  pl.blocks = (int)((N + rows - 1) / rows);
  if (S == 0) {
    // one activation tile: splits of about 8 k-steps; more tiles: about 1.5 workgroups
    // per CU (measured on MI355X over the Qwen3 projection shapes)
    if (pl.MT == 1) {
      const int per = std::max(1, 8 / pl.unit_steps);
      S = (pl.units + per - 1) / per;
    } else {
      S = (int)((400 + pl.blocks / 2) / pl.blocks);
    }
    if (S < 1) S = 1;
  }
  if (S > pl.units) S = pl.units;
  if ((int64_t)pl.blocks * pl.mtiles > kMaxCounters) S = 1;
  pl.S = S < 1 ? 1 : S;
  // x chunk: the split's whole range when it fits the LDS budget, in multiples of D
  const int64_t range = (int64_t)((pl.units + pl.S - 1) / pl.S) * pl.unit_steps;
  auto lds_for = [&](int64_t cs) { return (size_t)(M * (cs * kStepK + 8) * 2 + cs * 16 * pl.MT * 4); };
  int64_t cs = (range + pl.D - 1) / pl.D * pl.D;
  while (cs > pl.D && lds_for(cs) > (size_t)kLdsBudget) cs -= pl.D;
  pl.chunk_steps = (int)cs;
  pl.lds_bytes = lds_for(cs);
  pl.partial_bytes = pl.S > 1 ? (size_t)pl.S * M * N * 4 * pl.mtiles : 0;
  return pl;
}

template <int KIND, bool HZ, int SD, int MT, int NR, bool G1>
void launch_stream_g(const StreamParams& p, dim3 grid, size_t lds, hipStream_t st) {
  // the LDS limit is set once per kernel (thread-safe)
  static std::once_flag lds_once;
  std::call_once(lds_once, [&] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&wo_stream_kernel<KIND, HZ, SD, MT, NR, G1>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBudget);
  });
  hipLaunchKernelGGL((wo_stream_kernel<KIND, HZ, SD, MT, NR, G1>), grid, dim3(waves_for<MT>() * 64), lds, st, p);
}

// int4 with one-step (128-code) groups has its own instantiation
template <int KIND, bool HZ, int SD, int MT, int NR>
void launch_stream(const StreamParams& p, dim3 grid, size_t lds, hipStream_t st) {
  if (KIND == KIND_INT4 && p.group_steps == 1) launch_stream_g<KIND, HZ, SD, MT, NR, true>(p, grid, lds, st);
  else launch_stream_g<KIND, HZ, SD, MT, NR, false>(p, grid, lds, st);
}

template <int KIND, bool HZ, int SD>
void launch_mt(const StreamParams& p, const StreamPlan& pl, dim3 grid, hipStream_t st) {
  const size_t lds = pl.lds_bytes;
  switch (pl.MT * 4 + pl.NR) {
    case 5: launch_stream<KIND, HZ, SD, 1, 1>(p, grid, lds, st); break;
    case 6: launch_stream<KIND, HZ, SD, 1, 2>(p, grid, lds, st); break;
    case 8: launch_stream<KIND, HZ, SD, 1, 4>(p, grid, lds, st); break;
    case 9: launch_stream<KIND, HZ, SD, 2, 1>(p, grid, lds, st); break;
    case 10: launch_stream<KIND, HZ, SD, 2, 2>(p, grid, lds, st); break;
    case 13: launch_stream<KIND, HZ, SD, 3, 1>(p, grid, lds, st); break;
    case 14: launch_stream<KIND, HZ, SD, 3, 2>(p, grid, lds, st); break;
    case 17: launch_stream<KIND, HZ, SD, 4, 1>(p, grid, lds, st); break;
    default: launch_stream<KIND, HZ, SD, 4, 2>(p, grid, lds, st); break;
  }
}

template <int KIND, bool HZ>
void launch_sd(int sd, const StreamParams& p, const StreamPlan& pl, dim3 grid, hipStream_t st) {
  if (sd == MIQ_BF16) launch_mt<KIND, HZ, MIQ_BF16>(p, pl, grid, st);
  else if (sd == MIQ_F16) launch_mt<KIND, HZ, MIQ_F16>(p, pl, grid, st);
  else launch_mt<KIND, HZ, MIQ_F32>(p, pl, grid, st);
}

}  // namespace

// Workspace bytes for a weight-only GEMM: arrival counters, then [S][M][N] fp32 partials.
// int4 plans depend on the group size, so the size covers every group that divides K.
size_t wo_stream_workspace_bytes(int64_t M, int64_t N, int64_t K, int weight_bits) {
  if (M < 1 || M > 64 || N < 1 || K < kStepK) return kCounterBytes;
  const int steps = (int)(K / kStepK);
  size_t most = 0;
  for (int gs = 1; gs <= steps; ++gs) {
    if (steps % gs) continue;
    const StreamPlan pl = plan_stream(weight_bits == 4 ? KIND_INT4 : KIND_INT8, M, N, K, gs);
    if (pl.partial_bytes > most) most = pl.partial_bytes;
    if (weight_bits != 4) break;
  }
  return kCounterBytes + most;
}

int wo_stream_launch(int kind, const uint16_t* x, int64_t ldx, const uint8_t* w, int64_t ldw, const void* scale,
                     const void* zero, int sd, int group_steps, int64_t ngroups, uint16_t* y, int64_t ldy, int M,
                     int N, int K, void* workspace, size_t ws_bytes, hipStream_t st, const char* name) {
  const StreamPlan pl = plan_stream(kind, M, N, K, group_steps);
  MIQ_REQUIRE(pl.lds_bytes <= (size_t)kLdsBudget, "%s: no LDS plan for M=%d", name, M);
  MIQ_REQUIRE(pl.S == 1 || ((int64_t)pl.blocks * pl.mtiles <= kMaxCounters && pl.partial_bytes < (1u << 31)),
              "%s: N=%d too large for a split-K plan", name, N);
  MIQ_REQUIRE((int64_t)N * ldw < 0x7fff0000LL, "%s: weights of %lld bytes exceed 2 GiB", name, (long long)N * ldw);
  const size_t need = kCounterBytes + pl.partial_bytes;
  MIQ_REQUIRE(pl.S == 1 || (workspace != nullptr && ws_bytes >= need),
              "%s: workspace of %zu bytes needed (got %zu)", name, need, ws_bytes);
  StreamParams p{};
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
  p.S = pl.S;
  p.units = pl.units;
  p.unit_steps = pl.unit_steps;
  p.chunk_steps = pl.chunk_steps;
  p.wbytes = (int)((int64_t)N * ldw);
  const int esz = sd == MIQ_F32 ? 4 : 2;
  p.sbytes = kind == KIND_INT4 ? (int)(((int64_t)N * ngroups * esz + 3) & ~3LL) : 0;
  p.counters = static_cast<int*>(workspace);
  p.partial = workspace ? reinterpret_cast<float*>(static_cast<char*>(workspace) + kCounterBytes) : nullptr;
  const dim3 grid((unsigned)pl.blocks, (unsigned)pl.S, (unsigned)pl.mtiles);
  if (kind == KIND_INT8) launch_sd<KIND_INT8, false>(sd, p, pl, grid, st);
  else if (zero) launch_sd<KIND_INT4, true>(sd, p, pl, grid, st);
  else launch_sd<KIND_INT4, false>(sd, p, pl, grid, st);
  return check_launch(name);
}

}  // namespace miq
