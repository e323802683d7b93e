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
constexpr int kTileLds = 160 * 1024;       // gfx950 LDS per workgroup
constexpr int kCUs = 256;                  // MI355X compute units
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
  int wbytes, sbytes;
};

template <int KIND, bool HZ, int SD, int W, bool G1>
__global__ void __launch_bounds__(W * 64)
wo_tile_kernel(TileParams p) {
  constexpr int kThreads = W * 64, NS = kTileNS, XP = tile_xp<KIND>();
  constexpr int kStepBytes = KIND == KIND_INT4 ? kStepK / 2 : kStepK;  // per weight row
  extern __shared__ __align__(16) uint16_t lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, g = lane >> 4;
  const int M = p.M;
  MIQ_TRACE(0);

  // this wavefront's slice of K, in whole units (groups, or pairs of them)
  const int u0 = p.units * wv / W, u1 = p.units * (wv + 1) / W;
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

  // ---- then every weight and scale word of the slice
  const int n0 = blockIdx.x * p.rows;
  const int nrow = n0 + r;
  const int nrows = min(p.rows, p.N - n0);  // rows of this tile that exist
  // load h: lane 32 c2 + 4 rr + cl reads row 8h + rr, bytes 64 c2 + 16 cl of the k-step pair
  const int lrr = (lane >> 2) & 7, lcl = lane & 3, lc2 = lane >> 5;
  int woff[2], wok[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    woff[h] = min(n0 + 8 * h + lrr, p.N - 1) * (int)p.ldw + st0 * kStepBytes + lc2 * 64 + lcl * 16;
    wok[h] = (8 * h + lrr - nrows) >> 31;  // all ones for a row of the tile
  }
  const int bp_addr = (32 * (r >> 3) + 4 * (r & 7) + g) * 4;
  const int soff = (int)(min(nrow, p.N - 1) * p.ngroups + st0 / p.group_steps);
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
  if (KIND == KIND_INT8 && tid < M * 16) row_scale = load_sd_raw<SD>(p.scale, min(n0 + (tid & 15), p.N - 1));
  // int4: the scale (and zero) words of the slice's groups, at most NS of them, with two
  // 16-byte loads from the aligned word holding the first one. They are requested before
  // the weights: the multiply of k-step d then waits only for the weight loads up to d
  // (loads complete in issue order), not for the last one
  constexpr int esz = SD == MIQ_F32 ? 4 : 2;
  uint32_t sw[8], zw[8];
  const int sbase = r < nrows ? (soff * esz) & ~3 : kOut - 32;
  if (KIND == KIND_INT4) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const auto v = __builtin_amdgcn_raw_buffer_load_b128(srs, sbase + 16 * h, 0, 0);
      const uint4 u = *reinterpret_cast<const uint4*>(&v);
      sw[4 * h] = u.x; sw[4 * h + 1] = u.y; sw[4 * h + 2] = u.z; sw[4 * h + 3] = u.w;
      if (HZ) {
        const auto vz = __builtin_amdgcn_raw_buffer_load_b128(zrs, sbase + 16 * h, 0, 0);
        const uint4 uz = *reinterpret_cast<const uint4*>(&vz);
        zw[4 * h] = uz.x; zw[4 * h + 1] = uz.y; zw[4 * h + 2] = uz.z; zw[4 * h + 3] = uz.w;
      }
    }
  }
  // int4: raw loads of k-steps d, d + 1 (d even) in wq[d], wq[d + 1]; int8: wq[d][0..1]
  constexpr int NL = KIND == KIND_INT4 ? 1 : 2;
  uint4 wq[NS][NL];
#pragma unroll
  for (int d = 0; d < NS; ++d) {
    if (KIND == KIND_INT8 || (d & 1) == 0) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int kp = ((d + (KIND == KIND_INT4 ? lc2 : 0) - nsteps_v) >> 31) & wok[h];
        const int off = ((woff[h] + d * kStepBytes) & kp) | (kOut & ~kp);
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(wrs, off, 0, 2 /* nt */);
        if (KIND == KIND_INT4) wq[d + h][0] = *reinterpret_cast<const uint4*>(&v);
        else wq[d][h] = *reinterpret_cast<const uint4*>(&v);
      }
    }
  }
  // value of group e (0-based in the slice) from those words: for 16-bit scales the first
  // group sits in the high half of word 0 when soff is odd
  const bool odd = esz == 2 && (soff & 1);
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
  const int xstride = p.steps * kStepK + 8;
  float* xsum = reinterpret_cast<float*>(lds + M * xstride);
  for (int base = 0; base < npieces; base += XP * 64) {
    if (base != 0) load_x(base);
#pragma unroll
    for (int j = 0; j < XP; ++j) {
      if (base + j * 64 >= npieces) break;  // past the slice
      const int i = base + lane + j * 64;
      const int ic = min(i, npieces - 1);
      const int m = ic / scols, c = st0 * (kStepK / 8) + ic - m * scols;
      *reinterpret_cast<uint4*>(lds + m * xstride + c * 8) = KIND == KIND_INT4 ? permute_for_u4(xr[j]) : xr[j];
      // 16 consecutive lanes (one DPP row) hold the 16 pieces of one k-step of one row
      float sm = sum8_bf16(xr[j]);
      sm += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sm), 0x111, 0xf, 0xf, true));
      sm += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sm), 0x112, 0xf, 0xf, true));
      sm += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sm), 0x114, 0xf, 0xf, true));
      sm += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sm), 0x118, 0xf, 0xf, true));
      if (i < npieces && (c & 15) == 15) xsum[(c >> 4) * 16 + m] = sm * kXBias;
    }
  }
  // this wavefront's LDS writes are complete before its lanes read each other's
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_wave_barrier();
  MIQ_TRACE(2);

  // ---- multiply the slice. Per quantization group, T = sum_k x (128 + u) + kXBias * sum_k x
  // (two MFMA chains and the staged sums), and acc += s * T (+ z * sum_k x with zero points)
  const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
  f32x4 acc = z4, accg = z4, acc2 = z4, xsg = z4;
  int c_grp = 0, c_left = p.group_steps;
  const uint16_t* xrow = lds + min(r, M - 1) * xstride;
  uint4 wnext;
#pragma unroll
  for (int d = 0; d < NS; ++d) {
    if (d < nst) {
      const int kl = st0 + d;
      bf16x8 av[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint4 v = *reinterpret_cast<const uint4*>(xrow + a_off<KIND>(kl, g, j));
        av[j] = as_bf16x8(v.x, v.y, v.z, v.w);
      }
      const f32x4 xb = *reinterpret_cast<const f32x4*>(xsum + kl * 16 + g * 4);
      uint4 wl[2];
      if (KIND == KIND_INT8) {
        lanes_to_mfma(bp_addr, wq[d][0], wq[d][1], wl[0], wl[1]);
      } else if ((d & 1) == 0) {
        lanes_to_mfma(bp_addr, wq[d][0], wq[d + 1][0], wl[0], wnext);
      } else {
        wl[0] = wnext;
      }
      bf16x8 bv[4];
      unpack_b<KIND>(wl, bv);
      if (KIND == KIND_INT4 && G1) {
        // one-step groups: the first chain starts from the step's bias, the second from
        // zero, and the group ends here (scale and zero of group d: compile-time indices)
        accg = mfma(av[0], bv[0], xb);
        acc2 = mfma(av[1], bv[1], z4);
        accg = mfma(av[2], bv[2], accg);
        acc2 = mfma(av[3], bv[3], acc2);
        const float sc = group_value(sw, d);
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[v] = __builtin_fmaf(sc, accg[v] + acc2[v], acc[v]);
        if (HZ) {
          const float zq = group_value(zw, d) * (1.f / kXBias);
#pragma unroll
          for (int v = 0; v < 4; ++v) acc[v] = __builtin_fmaf(zq, xb[v], acc[v]);
        }
      } else {
        xsg += xb;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          f32x4& chain = (j & 1) ? acc2 : (KIND == KIND_INT4 ? accg : acc);
          chain = mfma(av[j], bv[j], chain);
        }
        if (KIND == KIND_INT4 && --c_left == 0) {  // end of a quantization group
          // group c_grp picked by a select chain (a run-time index into the word array
          // would spill it)
          float sc = group_value(sw, 0), zv = 0.f;
          if (HZ) zv = group_value(zw, 0);
#pragma unroll
          for (int e = 1; e < NS; ++e) {
            if (e > d) break;
            sc = c_grp == e ? group_value(sw, e) : sc;
            if (HZ) zv = c_grp == e ? group_value(zw, e) : zv;
          }
#pragma unroll
          for (int v = 0; v < 4; ++v) acc[v] = __builtin_fmaf(sc, accg[v] + acc2[v] + xsg[v], acc[v]);
          if (HZ) {
            const float zq = zv * (1.f / kXBias);
#pragma unroll
            for (int v = 0; v < 4; ++v) acc[v] = __builtin_fmaf(zq, xsg[v], acc[v]);
          }
          accg = z4;
          acc2 = z4;
          xsg = z4;
          ++c_grp;
          c_left = p.group_steps;
        }
      }
    }
  }
  if (KIND == KIND_INT8) {
#pragma unroll
    for (int v = 0; v < 4; ++v) acc[v] += acc2[v] + xsg[v];
  }

  MIQ_TRACE(3);
  // ---- add the W partial tiles in wavefront order: red [W][M][16] fp32 over the x area
  __syncthreads();  // every wavefront is done reading the activations
  float* red = reinterpret_cast<float*>(lds);
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int m = g * 4 + v;  // lane (r, g) holds y[4 g + v][n0 + r]
    if (m < M) red[(wv * M + m) * 16 + r] = acc[v];
  }
  __syncthreads();
  // kThreads >= 256 >= 16 M: one output per thread at most
  for (int t = tid; t < M * 16; t += kThreads) {
    const int m = t >> 4, n = n0 + (t & 15);
    if ((t & 15) >= nrows) continue;
    float o = 0.f;
#pragma unroll
    for (int w = 0; w < W; ++w) o += red[w * M * 16 + t];
    if (KIND == KIND_INT8)
      o = bf16_to_f32(f32_to_bf16(o)) * bf16_to_f32(f32_to_bf16(sd_to_f32<SD>(row_scale)));
    p.y[(int64_t)m * p.ldy + n] = f32_to_bf16(o);
  }
  MIQ_TRACE(4);
}

template <int KIND, bool HZ, int SD, int W, bool G1>
void launch_tile_g(const TileParams& p, unsigned blocks, size_t lds, hipStream_t st) {
  // the LDS limit is set once per kernel (thread-safe)
  static std::once_flag lds_once;
  std::call_once(lds_once, [&] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&wo_tile_kernel<KIND, HZ, SD, W, G1>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, kTileLds);
  });
  hipLaunchKernelGGL((wo_tile_kernel<KIND, HZ, SD, W, G1>), dim3(blocks), dim3(W * 64), lds, st, p);
}

// int4 with one-step (128-code) groups has its own instantiation
template <int KIND, bool HZ, int SD, int W>
void launch_tile(const TileParams& p, unsigned blocks, size_t lds, hipStream_t st) {
  if (KIND == KIND_INT4 && p.group_steps == 1) launch_tile_g<KIND, HZ, SD, W, true>(p, blocks, lds, st);
  else launch_tile_g<KIND, HZ, SD, W, false>(p, blocks, lds, st);
}

template <int KIND, bool HZ, int SD>
void launch_w(int W, const TileParams& p, unsigned blocks, size_t lds, hipStream_t st) {
  if (W == 4) launch_tile<KIND, HZ, SD, 4>(p, blocks, lds, st);
  else if (W == 8) launch_tile<KIND, HZ, SD, 8>(p, blocks, lds, st);
  else launch_tile<KIND, HZ, SD, 16>(p, blocks, lds, st);
}

template <int KIND, bool HZ>
void launch_tile_sd(int sd, int W, const TileParams& p, unsigned blocks, size_t lds, hipStream_t st) {
  if (sd == MIQ_BF16) launch_w<KIND, HZ, MIQ_BF16>(W, p, blocks, lds, st);
  else if (sd == MIQ_F16) launch_w<KIND, HZ, MIQ_F16>(W, p, blocks, lds, st);
  else launch_w<KIND, HZ, MIQ_F32>(W, p, blocks, lds, st);
}

}  // namespace

// The tile plan for (M, N, K): wavefronts per workgroup W (0 = the tile kernel does not
// apply: more than 16 rows, a slice longer than 8 k-steps, or activations too large for
// LDS), the unit of K slicing and the LDS bytes.
struct TilePlan {
  int W, units, unit_steps, rows;
  size_t lds_bytes;
};

static TilePlan plan_tile(int kind, int64_t M, int64_t N, int64_t K, int group_steps) {
  TilePlan pl{0, 0, 0, 0, 0};
  if (M < 1 || M > 16 || N < 1 || K < kStepK) return pl;
  if (tuning().wo_stream) return pl;  // force the streamed kernel (tuning, tests)
  // int8 with more than 4 rows: the streamed kernel (N = 19456, K = 2560 on MI355X: tile
  // kernel at M = 3 / 4 / 8 / 16 12.0 / 12.9 / 15.3 / 16.9 us, streamed 14.1 / 14.2 / 15.2 /
  // 17.0 us; the staged activations of a tile grow with M)
  if (kind == KIND_INT8 && M > 4) return pl;
  const int64_t steps = K / kStepK;
  int us = kind == KIND_INT4 ? group_steps : 1;
  // int4 slices start on an even k-step when they can (whole 128-byte lines per load)
  if (kind == KIND_INT4 && us % 2 == 1 && steps % (2 * us) == 0) us *= 2;
  const int64_t units = steps / us;
  if (us > kTileNS) return pl;
  const int64_t xbytes = M * (steps * kStepK + 8) * 2;
  // rows per tile: 16 (MIQ_WO_ROWS overrides, tuning). With per-wavefront activation
  // staging, 16-row tiles measured faster than fewer rows spread over every CU (INT4
  // N = 2560, K = 9728 on MI355X: M = 1 6.5 against 6.7 us with 10-row tiles, M = 8 10.7
  // against 11.1 us); before that change the 10-row tiles had been 4 % faster at M = 1.
  int rows = 16;
  if (tuning().wo_rows > 0) rows = std::max(1, std::min(16, tuning().wo_rows));
  const int64_t tiles = (N + rows - 1) / rows;
  for (int W : {4, 8, 16}) {
    if ((units + W - 1) / W * us > kTileNS) continue;
    const size_t lds = (size_t)std::max<int64_t>(xbytes, (int64_t)W * M * 16 * 4) + (size_t)steps * 16 * 4;
    if (lds > (size_t)kTileLds) return pl;
    // every tile should be resident at once (a second wave of workgroups would stage the
    // activations again): workgroups per CU from LDS and from 16 wavefronts per CU
    const int64_t per_cu = std::min<int64_t>((int64_t)kTileLds / (int64_t)lds, 16 / W);
    if (tiles > per_cu * kCUs * 5 / 4) return pl;
    pl.W = W;
    pl.units = (int)units;
    pl.unit_steps = us;
    pl.lds_bytes = lds;
    pl.rows = rows;
    return pl;
  }
  return pl;
}

// Launches the tile kernel when it applies (`launched` says whether it did); returns a
// MIQ_* status.
int wo_tile_launch(int kind, const uint16_t* x, int64_t ldx, const uint8_t* w, int64_t ldw, const void* scale,
                   const void* zero, int sd, int group_steps, int64_t ngroups, uint16_t* y, int64_t ldy, int M,
                   int N, int K, hipStream_t st, const char* name, bool& launched) {
  launched = false;
  const TilePlan pl = plan_tile(kind, M, N, K, group_steps);
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
  p.wbytes = (int)((int64_t)N * ldw);
  const int esz = sd == MIQ_F32 ? 4 : 2;
  p.sbytes = kind == KIND_INT4 ? (int)(((int64_t)N * ngroups * esz + 3) & ~3LL) : 0;
  const unsigned blocks = (unsigned)((N + pl.rows - 1) / pl.rows);
  if (kind == KIND_INT8) launch_tile_sd<KIND_INT8, false>(sd, pl.W, p, blocks, pl.lds_bytes, st);
  else if (zero) launch_tile_sd<KIND_INT4, true>(sd, pl.W, p, blocks, pl.lds_bytes, st);
  else launch_tile_sd<KIND_INT4, false>(sd, pl.W, p, blocks, pl.lds_bytes, st);
  launched = true;
  return check_launch(name);
}

}  // namespace miq
