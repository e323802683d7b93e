// Weight-only INT4 skinny GEMM (1 <= M <= 64) as panels of the weight matrix, gfx950:
//
//   y[m, n] = sum_k x[m, k] * W[n, k],  x bf16 [M, K],  W int4 [N, K/2] (+ group scales)
//
// The weight matrix is cut into panels of ROWS = 4 * NR * 16 rows (a row block) by at
// most kPanelSteps k-steps of 128 (one of S K-splits), and the activations into groups of
// MT * 16 rows; one workgroup of 4 wavefronts owns one (panel, activation group),
// wavefront w the panel's rows 16 NR w .. 16 NR (w + 1) - 1. The workgroups of one panel
// on its different activation groups have ids 8 apart: they run on the same XCD at about
// the same time and read the panel's weight lines from that XCD's L2 after the first
// fetch. Small workgroups (one 16-row activation group by default) let several share a CU,
// so one workgroup's multiply overlaps another's loads. A workgroup sees a single memory
// round trip:
//   * the M activation rows of its K range go from memory straight into LDS (buffer_load
//     ... lds, natural order), then every weight and scale load of the panel is issued at
//     once (NR * kPanelSteps 16-byte loads per lane, whole 128-byte lines in address
//     order), before anything waits;
//   * one LDS pass then puts the activations into the unpack order of the nibble codes and
//     forms the per-k-step sums that remove the +128 code offset;
//   * the multiply is the per-element math of the other weight-only kernels (wo_core.h):
//     codes unpacked to bf16 128 + u, v_mfma_f32_16x16x32_bf16 in fp32, per group
//     acc += s * (sum x (128 + u) + bias * sum x) [+ z * sum x].
// Split-K reduction without a serial tail: every workgroup stores its fp32 partial panel
// with agent-coherent (sc1) stores and bumps the arrival counter of its (row block,
// activation group); the S workgroups of row block rb + 1 on the same activation group
// then reduce row block rb, each one slice of its outputs, adding the S partials in split
// order (deterministic) and writing bf16. The grid carries one extra row block of
// reduce-only workgroups for the last row block. A reducer only ever waits for workgroups
// with lower ids (same activation group, lower panel), which were dispatched before it
// and never wait for it, so the wait cannot deadlock whatever the occupancy. The reducers
// reset the counters once they are all done, so every call leaves them at zero.
#include <algorithm>
#include <mutex>

#include "wo_core.h"

#ifndef MIQ_TRACE
#define MIQ_TRACE(point)  // per-workgroup timestamps in probe builds
#endif
// Ablation bits for timing probes, compiled in only with -DMIQ_PANEL_ABL=<bits> (the
// results are then wrong): 1 no reduction, 2 no partial stores, 4 no activation loads,
// 16 no multiply. The shipped library is built with 0.
#ifndef MIQ_PANEL_ABL
#define MIQ_PANEL_ABL 0
#endif

namespace miq {
namespace {

using namespace wo;

constexpr int kPanelWaves = 4;
constexpr int kPanelSteps = 8;            // k-steps one workgroup multiplies (all loads at once)
constexpr int kPanelLds = 159 * 1024;     // dynamic LDS per workgroup (160 KiB on gfx950, less the static LDS)
constexpr int kCUs = 256;                 // MI355X compute units
constexpr int kSpinLimit = 1 << 22;       // polls before a reducer gives up (never reached)

struct PanelParams {
  const uint16_t* x;
  int64_t ldx;
  const uint8_t* w;
  int64_t ldw;          // bytes per weight row (K / 2)
  const void* scale;
  const void* zero;
  int group_steps;      // k-steps per quantization group
  int64_t ngroups;      // groups per weight row
  uint16_t* y;
  int64_t ldy;
  int M, N;
  int blocks;           // row blocks that hold weights (the grid has one more when S > 1)
  int S;                // K splits
  int groups;           // activation groups of MT * 16 rows
  int panels;           // panels in the grid: (blocks + (S > 1)) * S
  int units, unit_steps;
  int xstride;          // LDS row pitch of the staged activations (elements)
  int wbytes, sbytes, xbytes;
  float* partial;       // [S][N][Mp] marked fp32 words (Mp = M rounded up to 4)
  int Mp;
  unsigned* error;      // device error word: set when a reducer gives up waiting
};
constexpr int kAbl = MIQ_PANEL_ABL;

// A partial as stored: the bits of v + 0 (so -0 becomes +0) with the sign bit flipped,
// which is never the all-zero word; the workspace holds zeros where no partial is pending.
__device__ inline uint32_t mark_partial(float v) { return __builtin_bit_cast(uint32_t, v + 0.f) ^ 0x80000000u; }
__device__ inline float unmark_partial(uint32_t w) { return __builtin_bit_cast(float, w ^ 0x80000000u); }

template <bool HZ, int SD, int MT, int NR, bool G1>
__device__ __forceinline__ void produce(const PanelParams& p, int rb, int s, int mg, uint16_t* lds) {
  constexpr int W = kPanelWaves, NS = kPanelSteps, ROWS = W * NR * 16, XR = MT * 16;
  constexpr int kStepBytes = kStepK / 2;
  constexpr float kXBias = HZ ? -128.f : -136.f;  // the MFMA sees codes as 128 + u
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, g = lane >> 4;
  const int m0 = mg * XR;                // first activation row of the group
  const int M = min(XR, p.M - m0);       // rows of the group
  const int u0 = (int)((int64_t)p.units * s / p.S), u1 = (int)((int64_t)p.units * (s + 1) / p.S);
  const int st0 = u0 * p.unit_steps, nst = (u1 - u0) * p.unit_steps;  // nst <= NS (host plan)

  // ---- 1. activations of the K range into LDS, row m at lds + m * xstride, natural order
  const int xcols = nst * (kStepK / 8);  // 16-byte pieces per row
  const int ipr = (xcols + 63) / 64;     // loads of up to 64 pieces per row
  const __amdgpu_buffer_rsrc_t xrs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(p.x), 0, p.xbytes, 0x00020000);
  for (int q = wv; q < ((kAbl & 4) ? 0 : M * ipr); q += W) {
    const int m = q / ipr, c0 = (q - m * ipr) * 64;
    if (c0 + lane < xcols)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          xrs, (__attribute__((address_space(3))) void*)(lds + m * p.xstride + c0 * 8), 16,
          (int)(((int64_t)(m0 + m) * p.ldx + (int64_t)st0 * kStepK + (c0 + lane) * 8) * 2), 0, 0, 0);
  }
  asm volatile("" ::: "memory");  // the weight loads below are issued after these
  MIQ_TRACE(1);

  // ---- 2. every weight and scale load of the panel
  const int n0 = rb * ROWS + wv * NR * 16;  // first row of this wavefront
  const int lrr = (lane >> 2) & 7, lcl = lane & 3, lc2 = lane >> 5;
  const int bp_addr = (32 * (r >> 3) + 4 * (r & 7) + g) * 4;
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(p.w), 0, p.wbytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p.scale), 0, p.sbytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t zrs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(HZ ? p.zero : p.scale), 0, p.sbytes, 0x00020000);
  constexpr int kOut = 0x7ffffff0;  // an offset outside every buffer: the load returns zeros
  int nsteps_v = nst;  // opaque per-lane value: requests past the range go to kOut by bit operations
  asm volatile("" : "+v"(nsteps_v));
  // scale (and zero) words of the range's groups, at most NS of them per row: two 16-byte
  // loads from the aligned word holding the first one (issued before the weights, so
  // waiting for them does not wait for the weights)
  constexpr int esz = SD == MIQ_F32 ? 4 : 2;
  uint32_t sw[NR][8], zw[NR][8];
  int sodd[NR];
#pragma unroll
  for (int t = 0; t < NR; ++t) {
    const int row = n0 + t * 16 + r;
    const int soff = (int)(min(row, p.N - 1) * p.ngroups + st0 / p.group_steps);
    sodd[t] = soff & 1;
    const int sbase = row < p.N ? (soff * esz) & ~3 : kOut - 32;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const auto v = __builtin_amdgcn_raw_buffer_load_b128(srs, sbase + 16 * h, 0, 0);
      const uint4 u = *reinterpret_cast<const uint4*>(&v);
      sw[t][4 * h] = u.x; sw[t][4 * h + 1] = u.y; sw[t][4 * h + 2] = u.z; sw[t][4 * h + 3] = u.w;
      if (HZ) {
        const auto vz = __builtin_amdgcn_raw_buffer_load_b128(zrs, sbase + 16 * h, 0, 0);
        const uint4 uz = *reinterpret_cast<const uint4*>(&vz);
        zw[t][4 * h] = uz.x; zw[t][4 * h + 1] = uz.y; zw[t][4 * h + 2] = uz.z; zw[t][4 * h + 3] = uz.w;
      }
    }
  }
  // load h of a pair of k-steps covers rows 8h .. 8h + 7 of a tile, 128 bytes each, in
  // address order within each 64-byte half (lane 32 c2 + 4 rr + cl: row 8h + rr, bytes
  // 64 c2 + 16 cl); the loads of pair d (d even) sit in wq[d][t] and wq[d + 1][t]. They
  // are issued pair by pair, so the multiply of the first pairs waits for those only.
  uint4 wq[NS][NR];
  int wbase[NR][2], wrok[NR][2];
#pragma unroll
  for (int t = 0; t < NR; ++t)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int row = n0 + t * 16 + 8 * h + lrr;
      wrok[t][h] = (row - p.N) >> 31;  // all ones for a row that exists
      wbase[t][h] = row * (int)p.ldw + st0 * kStepBytes + lc2 * 64 + lcl * 16;
    }
#pragma unroll
  for (int d = 0; d < NS; d += 2)
#pragma unroll
    for (int t = 0; t < NR; ++t)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int kp = ((d + lc2 - nsteps_v) >> 31) & wrok[t][h];
        const int off = ((wbase[t][h] + d * kStepBytes) & kp) | (kOut & ~kp);
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(wrs, off, 0, 0);  // default policy: the other activation groups re-read these lines from L2
        wq[d + h][t] = *reinterpret_cast<const uint4*>(&v);
      }
  // value of group e (0-based in the range) of tile t; 16-bit values start in the high half
  // of word 0 when the first group's element index is odd
  auto group_value = [&](const uint32_t* wds, int odd, int e) -> float {
    if constexpr (SD == MIQ_F32) {
      return __builtin_bit_cast(float, wds[e]);
    } else {
      const uint32_t even = (e & 1) ? (wds[e >> 1] >> 16) : (wds[e >> 1] & 0xffffu);
      const uint32_t oddv = ((e + 1) & 1) ? (wds[(e + 1) >> 1] >> 16) : (wds[(e + 1) >> 1] & 0xffffu);
      return sd_to_f32<SD>(odd ? oddv : even);
    }
  };

  // ---- 3. wait for this wavefront's activation loads (issued before the scale loads and
  // the NR * NS weight loads); after the barrier every wavefront's rows are in LDS
  constexpr int kLater = NR * NS + NR * 2 * (HZ ? 2 : 1);
  static_assert(kLater < 64, "vmcnt holds at most 63 outstanding loads");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kLater) : "memory");
  __syncthreads();
  MIQ_TRACE(2);
  MIQ_TRACE(3);
  // ---- 4. multiply: lane (r, g) accumulates y[16 mt + 4 g + v][n0 + 16 t + r]
  const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
  const bf16x8 ones = as_bf16x8(0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u);
  f32x4 acc[NR][MT], accg[NR][MT], acc2[NR][MT], xsg[MT];
#pragma unroll
  for (int t = 0; t < NR; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) { acc[t][mt] = z4; accg[t][mt] = z4; acc2[t][mt] = z4; }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) xsg[mt] = z4;
  int c_grp = 0, c_left = p.group_steps;
  uint4 wnext[NR];
  if (kAbl & 16) {  // ablation: the weights are consumed without a multiply
    uint32_t z = 0;
#pragma unroll
    for (int d = 0; d < NS; ++d)
#pragma unroll
      for (int t = 0; t < NR; ++t) z ^= wq[d][t].x ^ wq[d][t].y ^ wq[d][t].z ^ wq[d][t].w ^ sw[t][d & 7];
    acc[0][0][0] = __builtin_bit_cast(float, z);
  }
#pragma unroll
  for (int d = 0; d < NS; ++d) {
    if (d < nst && !(kAbl & 16)) {
      bf16x8 av[MT][4];
      f32x4 xb[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        // the A operand in the unpack order of the nibble codes (LDS holds natural order),
        // and kXBias times the sum of the step's activations per row, from an MFMA with a
        // ones operand: it lands in the accumulator layout (lane (r, g): rows 4 g + v)
        const uint16_t* row = lds + min(mt * 16 + r, M - 1) * p.xstride;
        f32x4 sums = z4;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint4 v = permute_for_u4(*reinterpret_cast<const uint4*>(row + a_off<KIND_INT4>(d, g, j)));
          av[mt][j] = as_bf16x8(v.x, v.y, v.z, v.w);
          sums = mfma(av[mt][j], ones, sums);
        }
#pragma unroll
        for (int v = 0; v < 4; ++v) xb[mt][v] = sums[v] * kXBias;
        if (!G1) xsg[mt] += xb[mt];
      }
#pragma unroll
      for (int t = 0; t < NR; ++t) {
        uint4 wl[1];
        if ((d & 1) == 0) lanes_to_mfma(bp_addr, wq[d][t], wq[d + 1][t], wl[0], wnext[t]);
        else wl[0] = wnext[t];
        bf16x8 bv[4];
        unpack_b<KIND_INT4>(wl, bv);
        if (G1) {
          // one-step groups: the first chain starts from the step's bias sums, the second
          // from zero, and the group ends with the step
          const float sc = group_value(sw[t], sodd[t], d);
          const float zq = HZ ? group_value(zw[t], sodd[t], d) * (1.f / kXBias) : 0.f;
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
              for (int v = 0; v < 4; ++v) acc[t][mt][v] = __builtin_fmaf(zq, xb[mt][v], acc[t][mt][v]);
            }
          }
        } else {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              f32x4& chain = (j & 1) ? acc2[t][mt] : accg[t][mt];
              chain = mfma(av[mt][j], bv[j], chain);
            }
        }
      }
      if (!G1 && --c_left == 0) {  // end of a quantization group (uniform)
#pragma unroll
        for (int t = 0; t < NR; ++t) {
          // group c_grp picked by a select chain (a run-time index into the word array
          // would move it to scratch)
          float sc = group_value(sw[t], sodd[t], 0), zv = HZ ? group_value(zw[t], sodd[t], 0) : 0.f;
#pragma unroll
          for (int e = 1; e < NS; ++e) {
            if (e > d) break;
            sc = c_grp == e ? group_value(sw[t], sodd[t], e) : sc;
            if (HZ) zv = c_grp == e ? group_value(zw[t], sodd[t], e) : zv;
          }
          const float zq = zv * (1.f / kXBias);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
            for (int v = 0; v < 4; ++v) {
              acc[t][mt][v] = __builtin_fmaf(sc, accg[t][mt][v] + acc2[t][mt][v] + xsg[mt][v], acc[t][mt][v]);
              if (HZ) acc[t][mt][v] = __builtin_fmaf(zq, xsg[mt][v], acc[t][mt][v]);
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
  }

  MIQ_TRACE(4);
  // ---- 5. the panel's result: bf16 when K is not split, else a marked fp32 partial.
  // Partials are [S][N][Mp]: lane (r, g) holds rows 4 g .. 4 g + 3 of column n of each
  // tile, one 16-byte store (a vector entirely past M is not stored).
  const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
      p.partial, 0, p.S > 1 ? (int)((int64_t)p.S * p.N * p.Mp * 4) : 0, 0x00020000);
#pragma unroll
  for (int t = 0; t < NR; ++t) {
    const int n = n0 + t * 16 + r;
    if (n >= p.N) continue;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int mv = mt * 16 + g * 4;  // first row of the lane's vector
      if (mv >= M) continue;
      if (p.S == 1) {
#pragma unroll
        for (int v = 0; v < 4; ++v)
          if (mv + v < M) p.y[(int64_t)(m0 + mv + v) * p.ldy + n] = f32_to_bf16(acc[t][mt][v]);
      } else if (!(kAbl & 2)) {
        const i32x4 w4 = {(int)mark_partial(acc[t][mt][0]), (int)mark_partial(acc[t][mt][1]),
                          (int)mark_partial(acc[t][mt][2]), (int)mark_partial(acc[t][mt][3])};
        __builtin_amdgcn_raw_buffer_store_b128(w4, prs, (int)((((int64_t)s * p.N + n) * p.Mp + m0 + mv) * 4), 0,
                                               16 /* sc1 */);
      } else if (acc[t][mt][0] == 1.2345f) {
        p.y[n] = 0;  // ablation runs: keep the multiply alive
      }
    }
  }
}

// Slice s of row block rb on activation group mg: vectors of 4 consecutive rows m of one
// column n, vector v = c * nm4 + j (column rb * ROWS + c, rows m0 + 4 j ..); this
// workgroup takes vectors [s V / S, (s + 1) V / S) and adds their S partials in split
// order. A partial word is there once it is non-zero (a
// producer never stores zero, see mark_partial); each word is read by this workgroup
// only, which sets it back to zero after reading it.
template <int MT, int NR>
__device__ __forceinline__ void reduce(const PanelParams& p, int rb, int s, int mg) {
  constexpr int kThreads = kPanelWaves * 64, ROWS = kPanelWaves * NR * 16, kChunk = 16;
  const int tid = threadIdx.x;
  const int m0 = mg * MT * 16;
  const int M = min(MT * 16, p.M - m0), S = p.S;  // rows of the group
  const int nm4 = (M + 3) / 4;  // row vectors per column
  const int V = ROWS * nm4;
  const int v0 = (int)((int64_t)V * s / S), v1 = (int)((int64_t)V * (s + 1) / S);
  const __amdgpu_buffer_rsrc_t prs =
      __builtin_amdgcn_make_buffer_rsrc(p.partial, 0, (int)((int64_t)S * p.N * p.Mp * 4), 0x00020000);
  const int sstride = p.N * p.Mp * 4;
  int spins = 0;
  bool gave_up = false;
  for (int v = v0 + tid; v < v1; v += kThreads) {
    const int c = v / nm4, m = (v - c * nm4) * 4, n = rb * ROWS + c;
    if (n >= p.N) continue;
    const int off = (n * p.Mp + m0 + m) * 4;
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int sp0 = 0; sp0 < S; sp0 += kChunk) {  // kChunk splits in flight, added in order
      uint4 t[kChunk];
      auto load = [&](int u) {
        const int so = sp0 + u < S ? off + (sp0 + u) * sstride : 0x7ffffff0;  // past the last split: zeros
        const auto w = __builtin_amdgcn_raw_buffer_load_b128(prs, so, 0, 16 /* sc1 */);
        t[u] = *reinterpret_cast<const uint4*>(&w);
      };
      auto pending = [&](int u) {
        return sp0 + u < S && (t[u].x == 0u || t[u].y == 0u || t[u].z == 0u || t[u].w == 0u);
      };
#pragma unroll
      for (int u = 0; u < kChunk; ++u) load(u);
      // producers still on their way: the missing ones are requested again together
      // (bounded: a reducer waits only for lower workgroup ids, which always finish)
      while (spins < kSpinLimit) {
        bool any = false;
#pragma unroll
        for (int u = 0; u < kChunk; ++u) any |= pending(u);
        if (!any) break;
        __builtin_amdgcn_s_sleep(1);
        ++spins;
#pragma unroll
        for (int u = 0; u < kChunk; ++u)
          if (pending(u)) load(u);
      }
      if (spins >= kSpinLimit) {
        // a producer never arrived (it cannot happen while every lower workgroup id runs
        // to completion): report it through the device error word and write NaN, never a
        // sum with a missing partial
        bool any = false;
#pragma unroll
        for (int u = 0; u < kChunk; ++u) any |= pending(u);
        gave_up |= any;
      }
      if (sp0 == 0) MIQ_TRACE(6);
      const i32x4 zero4 = {0, 0, 0, 0};
#pragma unroll
      for (int u = 0; u < kChunk; ++u) {
        if (sp0 + u >= S) break;
        o.x += unmark_partial(t[u].x);
        o.y += unmark_partial(t[u].y);
        o.z += unmark_partial(t[u].z);
        o.w += unmark_partial(t[u].w);
        __builtin_amdgcn_raw_buffer_store_b128(zero4, prs, off + (sp0 + u) * sstride, 0, 16 /* sc1 */);
      }
    }
    if (gave_up) {
      o = make_float4(__builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""));
      raise_device_error(p.error, MIQ_DEVERR_PANEL_WAIT);
    }
    uint16_t* yp = p.y + (int64_t)(m0 + m) * p.ldy + n;
    const float ov[4] = {o.x, o.y, o.z, o.w};
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (m + e < M) yp[(int64_t)e * p.ldy] = f32_to_bf16(ov[e]);
  }
}

template <bool HZ, int SD, int MT, int NR, bool G1>
__global__ void __launch_bounds__(kPanelWaves * 64)
wo_panel_kernel(PanelParams p) {
  extern __shared__ __align__(16) uint16_t lds[];
  // workgroup id -> (panel q, activation group mg): the groups of a panel are 8 ids apart
  // (same XCD), panels q and q + 1 are neighbours within each run of 8
  const int run = 8 * p.groups;
  const int id = blockIdx.x, rem = id % run;
  const int mg = rem / 8, q = (id / run) * 8 + rem % 8;
  if (q >= p.panels) return;
  const int rb = q / p.S, s = q - rb * p.S;
  MIQ_TRACE(0);
  if (rb < p.blocks) produce<HZ, SD, MT, NR, G1>(p, rb, s, mg, lds);
  MIQ_TRACE(5);
  if (p.S > 1 && rb >= 1 && !kAbl) reduce<MT, NR>(p, rb - 1, s, mg);
  MIQ_TRACE(7);
}

constexpr int kPanelNR = 2;  // weight tiles per wavefront: 128-row panels

template <bool HZ, int SD, int MT, bool G1>
void launch_g(const PanelParams& p, unsigned grid, size_t lds, hipStream_t st) {
  static std::once_flag lds_once;  // the LDS limit is set once per kernel (thread-safe)
  std::call_once(lds_once, [] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&wo_panel_kernel<HZ, SD, MT, kPanelNR, G1>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, kPanelLds);
  });
  hipLaunchKernelGGL((wo_panel_kernel<HZ, SD, MT, kPanelNR, G1>), dim3(grid), dim3(kPanelWaves * 64), lds, st, p);
}

template <bool HZ, int SD>
void launch_mt(int MT, const PanelParams& p, unsigned grid, size_t lds, hipStream_t st) {
  const bool g1 = p.group_steps == 1;
#define MIQ_PANEL(MTV) (g1 ? launch_g<HZ, SD, MTV, true>(p, grid, lds, st) : launch_g<HZ, SD, MTV, false>(p, grid, lds, st))
  switch (MT) {
    case 1: MIQ_PANEL(1); break;
    case 2: MIQ_PANEL(2); break;
    default: MIQ_PANEL(4); break;
  }
#undef MIQ_PANEL
}

}  // namespace

// The panel plan for an INT4 GEMM: K splits S (0 = the kernel does not apply), row
// blocks, the split unit and the LDS bytes.
struct PanelPlan {
  int S, blocks, units, unit_steps, xstride, MT, groups;
  size_t lds_bytes, partial_bytes;
};

PanelPlan plan_panel(int64_t M, int64_t N, int64_t K, int group_steps) {
  PanelPlan pl{};
  const Tuning& tu = tuning();
  if (tu.wo_panel == 0 || tu.wo_stream) return pl;
  // up to 16 rows the tile kernel (no K split, no cross-workgroup exchange) measured
  // faster on MI355X at the Qwen3 down_proj shape (M = 1: 6.6 against 11.7 us, M = 8:
  // 10.7 against 12.4 us); MIQ_WO_PANEL=1 takes the panel kernel there too
  if (tu.wo_panel < 0 && M <= 16) return pl;
  if (M < 1 || M > 64 || N < 1 || K < kStepK || group_steps > kPanelSteps) return pl;
  const int64_t steps = K / kStepK;
  constexpr int rows = kPanelWaves * kPanelNR * 16;
  const int64_t blocks = (N + rows - 1) / rows;
  // activation tiles of 16 rows per workgroup: 1 up to 32 rows, 2 above (MIQ_WO_PANEL_MT:
  // 1, 2 or 4). Measured at the Qwen3 down_proj shape on MI355X: M = 32 14.9 us with one
  // tile against 15.9 with two; M = 64 19.6 us with two against 23.3 with one, where the
  // 1008 workgroups of single tiles do not all fit the GPU at once
  int MT = M > 32 ? 2 : 1;
  if (tu.wo_panel_mt == 1 || tu.wo_panel_mt == 2 || tu.wo_panel_mt == 4) MT = tu.wo_panel_mt;
  MT = (int)std::min<int64_t>(MT, (M + 15) / 16);
  const int64_t groups = (M + 16 * MT - 1) / (16 * MT);
  if ((blocks + 1) * groups * 8 * rows >= (1LL << 31)) return pl;
  // splits start on a group boundary and, where the groups allow, on an even k-step
  // (whole 128-byte weight lines per load)
  int unit = group_steps;
  if (unit % 2 == 1 && steps % (2 * unit) == 0) unit *= 2;
  if (unit > kPanelSteps) unit = group_steps;
  const int64_t units = steps / unit;
  const int64_t per_max = kPanelSteps / unit;  // units one workgroup can take
  const int64_t s_min = (units + per_max - 1) / per_max;
  // about one panel per CU (producers plus the extra reduce-only row block), divided by
  // the activation tiles a workgroup takes (Qwen3 down_proj on MI355X, weights from HBM:
  // M = 64 with two tiles 18.9 us at 10 splits against 19.5 at 12 (0.1-0.2 us apart on another
  // box), 26.1-26.6 at 14-16; M = 32
  // with one tile 14.7-15.0 at 12 against 14.9-15.5 at 10)
  int64_t S = std::max<int64_t>(s_min, kCUs / ((blocks + 1) * MT));
  if (tu.wo_panel_s > 0) S = std::max<int64_t>(s_min, tu.wo_panel_s);
  S = std::min<int64_t>(S, units);
  if (s_min > units) return pl;
  const int64_t nst_max = (units + S - 1) / S * unit;
  const int64_t xstride = nst_max * kStepK + 8;
  const size_t lds = (size_t)(16 * MT * xstride * 2);
  if (lds > (size_t)kPanelLds) return pl;
  pl.S = (int)S;
  pl.blocks = (int)blocks;
  pl.units = (int)units;
  pl.unit_steps = unit;
  pl.xstride = (int)xstride;
  pl.MT = MT;
  pl.groups = (int)groups;
  pl.lds_bytes = lds;
  pl.partial_bytes = S > 1 ? (size_t)S * ((M + 3) / 4 * 4) * N * 4 : 0;
  return pl;
}

size_t wo_panel_partial_bytes(int64_t M, int64_t N, int64_t K) {
  size_t most = 0;
  const int64_t steps = K / kStepK;
  for (int gs = 1; gs <= kPanelSteps && gs <= steps; ++gs) {
    if (steps % gs) continue;
    const PanelPlan pl = plan_panel(M, N, K, gs);
    most = std::max(most, pl.partial_bytes);
  }
  return most;
}

// Launches the panel kernel when it applies (`launched` says whether it did); returns a
// MIQ_* status. The partials ([S][N][Mp] words, zero where none is pending) start at byte
// `skip` of the workspace, after the streamed kernel's counter area.
int wo_panel_launch(const uint16_t* x, int64_t ldx, const uint8_t* w, int64_t ldw, const void* scale,
                    const void* zero, int sd, int group_steps, int64_t ngroups, uint16_t* y, int64_t ldy, int M,
                    int N, int K, void* workspace, size_t ws_bytes, size_t skip, hipStream_t st,
                    const char* name, bool& launched) {
  launched = false;
  const PanelPlan pl = plan_panel(M, N, K, group_steps);
  if (pl.S == 0) return MIQ_OK;
  MIQ_REQUIRE((int64_t)N * ldw < 0x7fff0000LL, "%s: weights of %lld bytes exceed 2 GiB", name, (long long)N * ldw);
  MIQ_REQUIRE((int64_t)M * ldx * 2 < 0x7fff0000LL, "%s: activations exceed 2 GiB", name);
  MIQ_REQUIRE(pl.S == 1 || (workspace != nullptr && ws_bytes >= skip + pl.partial_bytes &&
                            pl.partial_bytes < (1u << 31)),
              "%s: workspace of %zu bytes needed (got %zu)", name, skip + pl.partial_bytes, ws_bytes);
  PanelParams p{};
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
  p.Mp = (M + 3) / 4 * 4;
  p.N = N;
  p.blocks = pl.blocks;
  p.S = pl.S;
  p.units = pl.units;
  p.unit_steps = pl.unit_steps;
  p.xstride = pl.xstride;
  p.wbytes = (int)((int64_t)N * ldw);
  const int esz = sd == MIQ_F32 ? 4 : 2;
  p.sbytes = (int)(((int64_t)N * ngroups * esz + 3) & ~3LL);
  p.xbytes = (int)((int64_t)M * ldx * 2);
  p.error = device_error_word();
  p.partial = workspace ? reinterpret_cast<float*>(static_cast<char*>(workspace) + skip) : nullptr;
  p.groups = pl.groups;
  p.panels = pl.S > 1 ? (pl.blocks + 1) * pl.S : pl.blocks;
  const unsigned grid = (unsigned)((p.panels + 7) / 8 * 8 * pl.groups);
  const int MT = pl.MT;
  if (zero) {
    if (sd == MIQ_BF16) launch_mt<true, MIQ_BF16>(MT, p, grid, pl.lds_bytes, st);
    else if (sd == MIQ_F16) launch_mt<true, MIQ_F16>(MT, p, grid, pl.lds_bytes, st);
    else launch_mt<true, MIQ_F32>(MT, p, grid, pl.lds_bytes, st);
  } else {
    if (sd == MIQ_BF16) launch_mt<false, MIQ_BF16>(MT, p, grid, pl.lds_bytes, st);
    else if (sd == MIQ_F16) launch_mt<false, MIQ_F16>(MT, p, grid, pl.lds_bytes, st);
    else launch_mt<false, MIQ_F32>(MT, p, grid, pl.lds_bytes, st);
  }
  launched = true;
  return check_launch(name);
}

}  // namespace miq
