// Weight-only quantized GEMM for decode (1 <= M <= 16 activation rows), one weight tile
// per workgroup:
//
//   y[m, n] = sum_k x[m, k] * W[n, k],  x bf16 [M, K],  W int8 [N, K] or int4 [N, K/2]
//
// A workgroup of W wavefronts owns one tile of R <= 16 weight rows over the whole K (the
// MFMA tile's other rows read nothing and are not written; R is 16 unless overridden);
// a launch has N / R workgroups of 4 to 16 wavefronts. The
// K range is cut into W slices of whole quantization groups, one per wavefront. Every
// wavefront requests its slice's activations, then its whole slice of weights (at most 8
// k-steps) and scales at once, so it sees one memory round trip instead of a ring of
// them. Each wavefront stages the activations of its own slice in LDS (the slices do not
// overlap, so no workgroup barrier precedes the multiply); the W partial tiles are added
// through LDS in wavefront order, so there is no split-K workspace, no cross-workgroup
// counter and no second round trip for partial sums. At M = 1 the time follows the
// k-steps per wavefront rather than the bytes per CU (on MI355X an M=1 launch takes about
// as long with 80 workgroups as with 256; halving K saves a third).
//
// INT4 at 7 to 10 rows (where a CU's staged activations outweigh its weights) takes the
// two-half plan: a workgroup owns two 16-row tiles over half of K, so each CU stages half
// the activations for the same weight bytes, and the two workgroups of a pair meet in one
// word per output of the caller's zeroed workspace. Each swaps its fp32 sum in with one
// agent-scope atomic exchange; the one that finds the other's sum adds the two (the same
// bits in either order), writes y and clears the word, so there is one round trip and no
// counter, and the workspace is all zeros again after the call. INT8 at 4 and 5 rows takes
// workgroups of two 16-row tiles over all of K, which share one staging of the activations
// (no exchange).
//
// Per-element math is the one of the streamed kernel (wo_stream.hip): codes unpack to
// bf16 128 + code, MFMA 16x16x32 bf16 with fp32 accumulation, and per quantization group
// acc += s * (sum x (128 + code) + bias * sum x) (bias -136 for symmetric int4 codes, -128
// with zero points, plus z * sum x); int8: acc - 128 * sum x, then the row scale.
//
// Weight loads read whole 128-byte lines: load h of the tile covers its rows 8h .. 8h + 7,
// 128 bytes each (two int4 k-steps or one int8 k-step), with four consecutive lanes on 64
// contiguous bytes (an order with four rows per four lanes measured 60 % slower from L2
// and 15 % slower from HBM on MI355X in a load-only test). A 32-lane swap and one lane
// gather per dword (lanes_to_mfma) then give every lane (g, r) row r, chunk g of each
// 64-byte half, the MFMA B layout.
#include <algorithm>
#include <cstdlib>

#include <mutex>

#include "miq_common.h"
#include "wo_core.h"

#ifndef MIQ_TRACE
#define MIQ_TRACE(point)  // per-wavefront timestamps in probe builds
#endif

namespace miq {
namespace {

using namespace wo;


constexpr int kTileNS = 8;                 // k-steps in flight per wavefront (all of its slice)
// k-steps a wavefront holds, by weight kind and row tiles: int8 with two row tiles holds 4
// (the weight registers of 8 would leave one wavefront per SIMD). Int4 with 10 (K = 9728
// then fits 8 wavefronts instead of 16) measured slower from M = 2 on (M = 1 / 2 / 4 / 6:
// 6.6 / 7.2-7.3 / 8.6-8.7 / 10.3-10.7 against 6.5-6.8 / 6.8-6.9 / 8.1-8.3 / 9.5-9.6 us)
constexpr int tile_ns(int kind, int nt) { return kind == KIND_INT8 && nt == 2 ? kTileNS / 2 : kTileNS; }
constexpr int kTileLds = 160 * 1024;       // gfx950 LDS per workgroup
constexpr int kCUs = 256;                  // MI355X compute units
// int4: rows of the two-half plan by default. INT4 N = 2560, K = 9728 on MI355X, weights
// read from HBM (rotating copies), one tile over all of K (M > 8: the streamed kernel)
// against two halves: M = 1 / 4 / 6 / 8 / 10 / 12 / 16 took 6.4 / 8.0 / 9.3 / 10.8 / 11.5 /
// 12.0 / 12.8 us against 7.6 / 8.7 / 9.5 / 10.25 / 11.3 / 12.3 / 13.9 us: the exchange costs
// about 1 us and pays at 8 to 10 rows, where a CU's staged activations outweigh its weights
constexpr int kPairMinM = 7, kPairMaxM = 10;
// int8: rows of the plan with two row tiles per workgroup over all of K. INT8 N = 19456,
// K = 2560 on MI355X (rotating weight copies), one tile per workgroup (M > 4: the streamed
// kernel) against two: M = 1 / 4 / 5 / 6 / 8 / 12 took 10.9-11.4 / 13.3-13.4 / 14.7-15.0 /
// 14.6-15.2 / 15.2-15.4 / 16.4-16.6 us against 12.3 / 13.1-13.2 / 13.6-13.9 / 14.9-15.0 /
// 15.9-16.1 / 18.2-18.3 us
constexpr int kInt8Tile2MinM = 4, kInt8Tile2MaxM = 5;
// activation pieces (16 B) per lane per round (int8 holds twice the weight registers):
// 12 x 64 pieces cover a wavefront's slice at M = 8 (8 rows x 6 k-steps) in one round;
// 16 measured slower (register pressure)
template <int KIND>
constexpr int tile_xp() { return KIND == KIND_INT4 ? 12 : 4; }

struct TileParams {
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
  int M, N, steps;      // steps = K / 128
  int rows;             // weight rows per tile (1..16)
  int units, unit_steps;
  int xsteps;           // k-steps of activations staged per workgroup (its K range)
  uint32_t* pair;       // two-half workgroups: [M][N] exchange words, all zero between calls
  int wbytes, sbytes;
};

// NT row tiles of 16 rows per workgroup; KS = 2 gives each tile two workgroups, one per
// half of K (workgroup 2 t + h takes half h of tile t), whose fp32 results meet in one
// exchange word per output (below).
template <int KIND, bool HZ, int SD, int W, bool G1, int NT, int KS>
__global__ void __launch_bounds__(W * 64)
wo_tile_kernel(TileParams p) {
  static_assert(KIND == KIND_INT4 || KS == 1, "int8 workgroups cover all of K");
  // k-steps in flight per wavefront: int8 with two row tiles holds 4 (the weight registers
  // of 8 would leave one wavefront per SIMD)
  constexpr int NS = tile_ns(KIND, NT);
  constexpr int kThreads = W * 64, XP = tile_xp<KIND>();
  constexpr int kStepBytes = KIND == KIND_INT4 ? kStepK / 2 : kStepK;  // per weight row
  extern __shared__ __align__(16) uint16_t lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, g = lane >> 4;
  const int M = p.M;
  MIQ_TRACE(0);

  // the workgroup's K range (units ua .. ub; LDS holds it from k-step kb on), then this
  // wavefront's slice of it, in whole units (groups, or pairs of them)
  const int half = KS == 2 ? (int)(blockIdx.x & 1) : 0;
  const int tile = KS == 2 ? (int)(blockIdx.x >> 1) : (int)blockIdx.x;
  const int ua = p.units * half / KS, ub = p.units * (half + 1) / KS;
  const int kb = ua * p.unit_steps;
  const int u0 = ua + (ub - ua) * wv / W, u1 = ua + (ub - ua) * (wv + 1) / W;
  const int st0 = u0 * p.unit_steps, nst = (u1 - u0) * p.unit_steps;

  // ---- activation loads first: each wavefront stages the M rows of its own slice of K
  // (the slices do not overlap, so no barrier is needed before the multiply), round 0
  // into registers
  const int scols = nst * (kStepK / 8);  // 16-byte pieces per activation row in the slice
  const int npieces = M * scols;
  const int xld = (int)(p.ldx / 8);
  const uint4* xsrc = reinterpret_cast<const uint4*>(p.x);
  uint4 xr[XP];
  // rounds of XP x 64 pieces; pieces j of a round past the slice are not loaded (a
  // uniform branch). Piece i: row i / scols, column st0 * 16 + i % scols.
  auto load_x = [&](int base) {
#pragma unroll
    for (int j = 0; j < XP; ++j) {
      if (base + j * 64 < npieces) {
        const int i = min(base + lane + j * 64, npieces - 1);
        const int m = i / scols, c = st0 * (kStepK / 8) + i - m * scols;
        xr[j] = xsrc[(int64_t)m * xld + c];
      }
    }
  };
  load_x(0);
  MIQ_TRACE(5);

  // ---- then every weight and scale word of the slice (row tile t: rows n0 + 16 t ..)
  const int n0 = tile * p.rows * NT;
  int nrows[NT];  // rows of each row tile that exist
#pragma unroll
  for (int t = 0; t < NT; ++t) nrows[t] = min(p.rows, p.N - n0 - 16 * t);
  // load h: lane 32 c2 + 4 rr + cl reads row 8h + rr, bytes 64 c2 + 16 cl of the k-step pair
  const int lrr = (lane >> 2) & 7, lcl = lane & 3, lc2 = lane >> 5;
  int woff[NT][2], wok[NT][2], soff[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      woff[t][h] = min(n0 + 16 * t + 8 * h + lrr, p.N - 1) * (int)p.ldw + st0 * kStepBytes + lc2 * 64 + lcl * 16;
      wok[t][h] = (8 * h + lrr - nrows[t]) >> 31;  // all ones for a row of the tile
    }
    soff[t] = (int)(min(n0 + 16 * t + r, p.N - 1) * p.ngroups + st0 / p.group_steps);
  }
  const int bp_addr = (32 * (r >> 3) + 4 * (r & 7) + g) * 4;
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(p.w), 0, p.wbytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p.scale), 0, p.sbytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t zrs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(HZ ? p.zero : p.scale), 0, p.sbytes, 0x00020000);
  constexpr int kOut = 0x7ffffff0;  // an offset outside every buffer: the load returns zeros
  // steps of the slice as an opaque per-lane value: loads past it are steered to kOut with
  // bit operations (a select would become a branch around each load)
  int nsteps_v = nst;
  asm volatile("" : "+v"(nsteps_v));
  // int8: the row scale of the output this thread writes at the end (thread t < 16 M
  // writes row n0 + t % 16), requested now rather than after the reduction
  uint32_t row_scale = 0;
  if (KIND == KIND_INT8 && NT == 1 && tid < M * 16) row_scale = load_sd_raw<SD>(p.scale, min(n0 + (tid & 15), p.N - 1));
  // int4: the scale (and zero) words of the slice's groups, at most NS of them, with two
  // 16-byte loads from the aligned word holding the first one. They are requested before
  // the weights: the multiply of k-step d then waits only for the weight loads up to d
  // (loads complete in issue order), not for the last one
  constexpr int esz = SD == MIQ_F32 ? 4 : 2;
  // words of the slice's group values: NS fp32 words, or up to NS / 2 + 1 words of 16-bit
  // values (the first may sit in the high half), in 16-byte loads
  constexpr int kSW = SD == MIQ_F32 ? (NS + 3) / 4 * 4 : 8;
  uint32_t sw[NT][kSW], zw[NT][kSW];
  if (KIND == KIND_INT4) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int sbase = r < nrows[t] ? (soff[t] * esz) & ~3 : kOut - 64;
#pragma unroll
      for (int h = 0; h < kSW / 4; ++h) {
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
  }
  // int4: raw loads of k-steps d, d + 1 (d even) in wq[t][d], wq[t][d + 1]; int8: wq[t][d][0..1]
  constexpr int NL = KIND == KIND_INT4 ? 1 : 2;
  uint4 wq[NT][NS][NL];
#pragma unroll
  for (int d = 0; d < NS; ++d) {
    if (KIND == KIND_INT8 || (d & 1) == 0) {
#pragma unroll
      for (int t = 0; t < NT; ++t) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int kp = ((d + (KIND == KIND_INT4 ? lc2 : 0) - nsteps_v) >> 31) & wok[t][h];
          const int off = ((woff[t][h] + d * kStepBytes) & kp) | (kOut & ~kp);
          const auto v = __builtin_amdgcn_raw_buffer_load_b128(wrs, off, 0, 2 /* nt */);
          if (KIND == KIND_INT4) wq[t][d + h][0] = *reinterpret_cast<const uint4*>(&v);
          else wq[t][d][h] = *reinterpret_cast<const uint4*>(&v);
        }
      }
    }
  }
  // value of group e (0-based in the slice) from those words: for 16-bit scales the first
  // group sits in the high half of word 0 when soff is odd (the same for every row tile:
  // their offsets differ by 16 rows of ngroups words)
  const bool odd = esz == 2 && (soff[0] & 1);
  auto group_value = [&](const uint32_t* wds, int e) -> float {
    if constexpr (SD == MIQ_F32) {
      return __builtin_bit_cast(float, wds[e]);
    } else {
      const uint32_t even = (e & 1) ? (wds[e >> 1] >> 16) : (wds[e >> 1] & 0xffffu);
      const uint32_t oddv = ((e + 1) & 1) ? (wds[(e + 1) >> 1] >> 16) : (wds[(e + 1) >> 1] & 0xffffu);
      return sd_to_f32<SD>(odd ? oddv : even);
    }
  };

  MIQ_TRACE(1);
  // ---- stage the activations: LDS x [M][K + 8] bf16 (int4: pieces permuted for the
  // unpack order), then xsum [steps][16] fp32, the sum of each row over each k-step times
  // the code bias kXBias (the MFMA sees codes as 128 + u; symmetric int4 weights are u - 8)
  constexpr float kXBias = KIND == KIND_INT4 && !HZ ? -136.f : -128.f;
  const int xstride = p.xsteps * kStepK + 8;
  float* xsum = reinterpret_cast<float*>(lds + M * xstride);
  const int kbc = kb * (kStepK / 8);  // the first 16-byte column staged
  for (int base = 0; base < npieces; base += XP * 64) {
    if (base != 0) load_x(base);
#pragma unroll
    for (int j = 0; j < XP; ++j) {
      if (base + j * 64 >= npieces) break;  // past the slice
      const int i = base + lane + j * 64;
      const int ic = min(i, npieces - 1);
      const int m = ic / scols, c = st0 * (kStepK / 8) + ic - m * scols;
      *reinterpret_cast<uint4*>(lds + m * xstride + (c - kbc) * 8) = KIND == KIND_INT4 ? permute_for_u4(xr[j]) : xr[j];
      // 16 consecutive lanes (one DPP row) hold the 16 pieces of one k-step of one row
      float sm = sum8_bf16(xr[j]);
      sm += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sm), 0x111, 0xf, 0xf, true));
      sm += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sm), 0x112, 0xf, 0xf, true));
      sm += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sm), 0x114, 0xf, 0xf, true));
      sm += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sm), 0x118, 0xf, 0xf, true));
      if (i < npieces && (c & 15) == 15) xsum[((c - kbc) >> 4) * 16 + m] = sm * kXBias;
    }
  }
  // this wavefront's LDS writes are complete before its lanes read each other's
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_wave_barrier();
  MIQ_TRACE(2);

  // ---- multiply the slice. Per quantization group, T = sum_k x (128 + u) + kXBias * sum_k x
  // (two MFMA chains and the staged sums), and acc += s * T (+ z * sum_k x with zero points);
  // the row tiles share the activation fragments
  const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
  f32x4 acc[NT], accg[NT], acc2[NT], xsg = z4;
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = accg[t] = acc2[t] = z4;
  int c_grp = 0, c_left = p.group_steps;
  const uint16_t* xrow = lds + min(r, M - 1) * xstride;
  uint4 wnext[NT];
#pragma unroll
  for (int d = 0; d < NS; ++d) {
    if (d < nst) {
      const int kl = st0 + d - kb;  // k-step within the staged range
      bf16x8 av[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint4 v = *reinterpret_cast<const uint4*>(xrow + a_off<KIND>(kl, g, j));
        av[j] = as_bf16x8(v.x, v.y, v.z, v.w);
      }
      const f32x4 xb = *reinterpret_cast<const f32x4*>(xsum + kl * 16 + g * 4);
      if (!(KIND == KIND_INT4 && G1)) xsg += xb;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        uint4 wl[2];
        if (KIND == KIND_INT8) {
          lanes_to_mfma(bp_addr, wq[t][d][0], wq[t][d][1], wl[0], wl[1]);
        } else if ((d & 1) == 0) {
          lanes_to_mfma(bp_addr, wq[t][d][0], wq[t][d + 1][0], wl[0], wnext[t]);
        } else {
          wl[0] = wnext[t];
        }
        bf16x8 bv[4];
        unpack_b<KIND>(wl, bv);
        if (KIND == KIND_INT4 && G1) {
          // one-step groups: the first chain starts from the step's bias, the second from
          // zero, and the group ends here (scale and zero of group d: compile-time indices)
          accg[t] = mfma(av[0], bv[0], xb);
          acc2[t] = mfma(av[1], bv[1], z4);
          accg[t] = mfma(av[2], bv[2], accg[t]);
          acc2[t] = mfma(av[3], bv[3], acc2[t]);
          const float sc = group_value(sw[t], d);
#pragma unroll
          for (int v = 0; v < 4; ++v) acc[t][v] = __builtin_fmaf(sc, accg[t][v] + acc2[t][v], acc[t][v]);
          if (HZ) {
            const float zq = group_value(zw[t], d) * (1.f / kXBias);
#pragma unroll
            for (int v = 0; v < 4; ++v) acc[t][v] = __builtin_fmaf(zq, xb[v], acc[t][v]);
          }
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            f32x4& chain = (j & 1) ? acc2[t] : (KIND == KIND_INT4 ? accg[t] : acc[t]);
            chain = mfma(av[j], bv[j], chain);
          }
        }
      }
      if (KIND == KIND_INT4 && !G1 && --c_left == 0) {  // end of a quantization group
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          // group c_grp picked by a select chain (a run-time index into the word array
          // would spill it)
          float sc = group_value(sw[t], 0), zv = 0.f;
          if (HZ) zv = group_value(zw[t], 0);
#pragma unroll
          for (int e = 1; e < NS; ++e) {
            if (e > d) break;
            sc = c_grp == e ? group_value(sw[t], e) : sc;
            if (HZ) zv = c_grp == e ? group_value(zw[t], e) : zv;
          }
#pragma unroll
          for (int v = 0; v < 4; ++v) acc[t][v] = __builtin_fmaf(sc, accg[t][v] + acc2[t][v] + xsg[v], acc[t][v]);
          if (HZ) {
            const float zq = zv * (1.f / kXBias);
#pragma unroll
            for (int v = 0; v < 4; ++v) acc[t][v] = __builtin_fmaf(zq, xsg[v], acc[t][v]);
          }
          accg[t] = z4;
          acc2[t] = z4;
        }
        xsg = z4;
        ++c_grp;
        c_left = p.group_steps;
      }
    }
  }
  if (KIND == KIND_INT8) {
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[t][v] += acc2[t][v] + xsg[v];
  }

  MIQ_TRACE(3);
  // ---- add the W partial tiles in wavefront order: red [W][M][16 NT] fp32 over the x area
  constexpr int kCols = 16 * NT;
  __syncthreads();  // every wavefront is done reading the activations
  float* red = reinterpret_cast<float*>(lds);
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int m = g * 4 + v;  // lane (r, g) holds y[4 g + v][n0 + 16 t + r]
      if (m < M) red[(wv * M + m) * kCols + 16 * t + r] = acc[t][v];
    }
  __syncthreads();
  for (int t = tid; t < M * kCols; t += kThreads) {
    const int m = t / kCols, col = t % kCols, n = n0 + col;
    if ((col & 15) >= (col >= 16 ? nrows[NT - 1] : nrows[0])) continue;
    float o = 0.f;
#pragma unroll
    for (int w = 0; w < W; ++w) o += red[w * M * kCols + t];
    if (KS == 2) {
      // the two halves of K meet in one word per output: each workgroup swaps in its sum,
      // marked so that it is never the all-zero word (the bits of o with the sign flipped,
      // -0 taken as +0). The first to arrive finds zero and is done; the second finds the
      // other half, adds (a + b == b + a, so the result does not depend on the order of
      // arrival), writes y and clears the word for the next call.
      uint32_t bits = __builtin_bit_cast(uint32_t, o);
      bits = bits == 0x80000000u ? 0u : bits;
      uint32_t* word = p.pair + (int64_t)m * p.N + n;
      const uint32_t other = __hip_atomic_exchange(word, bits ^ 0x80000000u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (other == 0u) continue;
      o += __builtin_bit_cast(float, other ^ 0x80000000u);
      __hip_atomic_store(word, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (KIND == KIND_INT8) {
      const uint32_t rs = NT == 1 ? row_scale : load_sd_raw<SD>(p.scale, n);
      o = bf16_to_f32(f32_to_bf16(o)) * bf16_to_f32(f32_to_bf16(sd_to_f32<SD>(rs)));
    }
    p.y[(int64_t)m * p.ldy + n] = f32_to_bf16(o);
  }
  MIQ_TRACE(4);
}

template <int KIND, bool HZ, int SD, int W, bool G1, int NT, int KS>
void launch_tile_g(const TileParams& p, unsigned blocks, size_t lds, hipStream_t st) {
  // the LDS limit is set once per kernel (thread-safe)
  static std::once_flag lds_once;
  std::call_once(lds_once, [&] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&wo_tile_kernel<KIND, HZ, SD, W, G1, NT, KS>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, kTileLds);
  });
  hipLaunchKernelGGL((wo_tile_kernel<KIND, HZ, SD, W, G1, NT, KS>), dim3(blocks), dim3(W * 64), lds, st, p);
}

// int4 with one-step (128-code) groups has its own instantiation; int4 workgroups can hold
// two row tiles over half of K each, int8 workgroups two row tiles over all of K (shape =
// row tiles x halves of K: 1, 2 or 4)
template <int KIND, bool HZ, int SD, int W>
void launch_tile(int shape, const TileParams& p, unsigned blocks, size_t lds, hipStream_t st) {
  if constexpr (KIND == KIND_INT8) {
    if (shape == 2) {  // two row tiles over all of K
      launch_tile_g<KIND, HZ, SD, W, false, 2, 1>(p, blocks, lds, st);
      return;
    }
  }
  if constexpr (KIND == KIND_INT4) {
    if (shape == 4) {  // two row tiles, two halves of K
      if (p.group_steps == 1) launch_tile_g<KIND, HZ, SD, W, true, 2, 2>(p, blocks, lds, st);
      else launch_tile_g<KIND, HZ, SD, W, false, 2, 2>(p, blocks, lds, st);
      return;
    }
    if (p.group_steps == 1) {
      launch_tile_g<KIND, HZ, SD, W, true, 1, 1>(p, blocks, lds, st);
      return;
    }
  }
  launch_tile_g<KIND, HZ, SD, W, false, 1, 1>(p, blocks, lds, st);
}

template <int KIND, bool HZ, int SD>
void launch_w(int W, int shape, const TileParams& p, unsigned blocks, size_t lds, hipStream_t st) {
  if (W == 4) launch_tile<KIND, HZ, SD, 4>(shape, p, blocks, lds, st);
  else if (W == 8) launch_tile<KIND, HZ, SD, 8>(shape, p, blocks, lds, st);
  else launch_tile<KIND, HZ, SD, 16>(shape, p, blocks, lds, st);
}

template <int KIND, bool HZ>
void launch_tile_sd(int sd, int W, int shape, const TileParams& p, unsigned blocks, size_t lds, hipStream_t st) {
  if (sd == MIQ_BF16) launch_w<KIND, HZ, MIQ_BF16>(W, shape, p, blocks, lds, st);
  else if (sd == MIQ_F16) launch_w<KIND, HZ, MIQ_F16>(W, shape, p, blocks, lds, st);
  else launch_w<KIND, HZ, MIQ_F32>(W, shape, p, blocks, lds, st);
}

}  // namespace

// The tile plan for (M, N, K): wavefronts per workgroup W (0 = the tile kernel does not
// apply: more than 16 rows, a slice longer than 8 k-steps, or activations too large for
// LDS), the unit of K slicing, row tiles per workgroup (nt = 2: two 16-row tiles over
// half of K each, a pair of workgroups per 32 rows), the staged k-steps and the LDS bytes.
struct TilePlan {
  int W, units, unit_steps, rows, nt, ks, xsteps;
  size_t lds_bytes;
  unsigned blocks;
};

static TilePlan plan_tile(int kind, int64_t M, int64_t N, int64_t K, int group_steps, bool pair_ok) {
  TilePlan pl{};
  if (M < 1 || M > 16 || N < 1 || K < kStepK) return pl;
  if (tuning().wo_stream) return pl;  // force the streamed kernel (tuning, tests)
  // int8 with more than 4 rows: the streamed kernel (N = 19456, K = 2560 on MI355X: tile
  // kernel at M = 3 / 4 / 8 / 16 12.0 / 12.9 / 15.3 / 16.9 us, streamed 14.1 / 14.2 / 15.2 /
  // 17.0 us; the staged activations of a tile grow with M)
  // int8 at 4 and 5 rows: workgroups of two 16-row tiles share one staging of the
  // activations (half the staged bytes per weight byte)
  const int t2 = tuning().wo_int8_tile2_min_m;  // MIQ_WO_INT8_TILE2_MIN_M: from that M up to 16
  const bool int8_two = kind == KIND_INT8 && t2 >= 0 && (t2 > 0 ? M >= t2 : (M >= kInt8Tile2MinM && M <= kInt8Tile2MaxM));
  if (kind == KIND_INT8 && M > 4 && !int8_two) return pl;
  const int64_t steps = K / kStepK;
  int us = kind == KIND_INT4 ? group_steps : 1;
  // int4 slices start on an even k-step when they can (whole 128-byte lines per load)
  if (kind == KIND_INT4 && us % 2 == 1 && steps % (2 * us) == 0) us *= 2;
  const int64_t units = steps / us;
  if (us > kTileNS) return pl;
  // int4 from pair_min_m rows on: 32-row workgroups over half of K each. Every CU then
  // stages half the activations of the one-tile plan (at M = 8 those are twice a tile's
  // weight bytes and bound the launch), and the halves meet in one exchange word per
  // output (which needs the caller's workspace)
  const bool forced = tuning().wo_pair_min_m > 0;  // MIQ_WO_PAIR_MIN_M: from that M up to 16
  const bool pair_m = forced ? M >= tuning().wo_pair_min_m : (M >= kPairMinM && M <= kPairMaxM);
  const int ks = kind == KIND_INT4 && pair_ok && units >= 2 && pair_m && tuning().wo_pair_min_m >= 0 ? 2 : 1;
  // (two row tiles per workgroup: 16-row pairs, 320 workgroups, measured 11.1 against
  // 9.6 us at M = 8)
  const int nt = int8_two ? 2 : ks;
  const int ns = tile_ns(kind, nt);  // k-steps per wavefront at most
  const int64_t xsteps = (units + ks - 1) / ks * us;  // k-steps staged per workgroup
  const int64_t xbytes = M * (xsteps * kStepK + 8) * 2;
  // rows per tile: 16 (MIQ_WO_ROWS overrides, tuning). With per-wavefront activation
  // staging, 16-row tiles measured faster than fewer rows spread over every CU (INT4
  // N = 2560, K = 9728 on MI355X: M = 1 6.5 against 6.7 us with 10-row tiles, M = 8 10.7
  // against 11.1 us); before that change the 10-row tiles had been 4 % faster at M = 1.
  int rows = 16;
  if (nt == 1 && tuning().wo_rows > 0) rows = std::max(1, std::min(16, tuning().wo_rows));
  const int64_t blocks = ks * ((N + rows * nt - 1) / (rows * nt));
  const int64_t wunits = (units + ks - 1) / ks;  // units per workgroup, at most
  for (int W : {4, 8, 16}) {
    if ((wunits + W - 1) / W * us > ns || W < tuning().wo_tile_min_w) continue;
    const size_t lds = (size_t)std::max<int64_t>(xbytes, (int64_t)W * M * 16 * nt * 4) + (size_t)xsteps * 16 * 4;
    if (lds > (size_t)kTileLds) return pl;
    // every tile should be resident at once (a second wave of workgroups would stage the
    // activations again): workgroups per CU from LDS and from 16 wavefronts per CU
    const int64_t per_cu = std::min<int64_t>((int64_t)kTileLds / (int64_t)lds, 16 / W);
    if (blocks > per_cu * kCUs * 5 / 4) return pl;
    pl.W = W;
    pl.units = (int)units;
    pl.unit_steps = us;
    pl.lds_bytes = lds;
    pl.rows = rows;
    pl.nt = nt;
    pl.ks = ks;
    pl.xsteps = (int)xsteps;
    pl.blocks = (unsigned)blocks;
    return pl;
  }
  return pl;
}

// Bytes of exchange words the two-half int4 plan needs: one fp32 word per output.
size_t wo_tile_pair_bytes(int64_t M, int64_t N) { return M >= 1 && M <= 16 ? (size_t)(M * N * 4) : 0; }

// Launches the tile kernel when it applies (`launched` says whether it did); returns a
// MIQ_* status. `pair` / `pair_bytes`: zeroed exchange words from the caller's workspace
// (may be null; the two-half plan then does not apply).
int wo_tile_launch(int kind, const uint16_t* x, int64_t ldx, const uint8_t* w, int64_t ldw, const void* scale,
                   const void* zero, int sd, int group_steps, int64_t ngroups, uint16_t* y, int64_t ldy, int M,
                   int N, int K, void* pair, size_t pair_bytes, hipStream_t st, const char* name, bool& launched) {
  launched = false;
  const bool pair_ok = pair != nullptr && pair_bytes >= wo_tile_pair_bytes(M, N) &&
                       (reinterpret_cast<uintptr_t>(pair) & 3) == 0;
  const TilePlan pl = plan_tile(kind, M, N, K, group_steps, pair_ok);
  if (pl.W == 0) return MIQ_OK;
  MIQ_REQUIRE((int64_t)N * ldw < 0x7fff0000LL, "%s: weights of %lld bytes exceed 2 GiB", name, (long long)N * ldw);
  TileParams p{};
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
  p.steps = K / kStepK;
  p.units = pl.units;
  p.unit_steps = pl.unit_steps;
  p.rows = pl.rows;
  p.xsteps = pl.xsteps;
  p.pair = pl.ks == 2 ? static_cast<uint32_t*>(pair) : nullptr;
  p.wbytes = (int)((int64_t)N * ldw);
  const int esz = sd == MIQ_F32 ? 4 : 2;
  p.sbytes = kind == KIND_INT4 ? (int)(((int64_t)N * ngroups * esz + 3) & ~3LL) : 0;
  if (kind == KIND_INT8) launch_tile_sd<KIND_INT8, false>(sd, pl.W, pl.nt, p, pl.blocks, pl.lds_bytes, st);
  else if (zero) launch_tile_sd<KIND_INT4, true>(sd, pl.W, pl.nt * pl.ks, p, pl.blocks, pl.lds_bytes, st);
  else launch_tile_sd<KIND_INT4, false>(sd, pl.W, pl.nt * pl.ks, p, pl.blocks, pl.lds_bytes, st);
  launched = true;
  return check_launch(name);
}

}  // namespace miq
