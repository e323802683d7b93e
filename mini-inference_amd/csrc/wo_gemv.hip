// Weight-only quantized GEMV for the smallest decode batches (M = 1 by default, at most
// 2 activation rows), gfx950:
//
//   y[m, n] = sum_k x[m, k] * W[n, k],  x bf16 [M, K],  W int4 [N, K/2] or int8 [N, K]
//
// At M = 1 the work is one streaming read of the weights; what limits a tiled kernel is
// the number of CUs that issue loads and the per-wavefront chain of round trips, not the
// multiply. This kernel therefore reads the weight matrix as one contiguous stream:
//   * wavefront v of the launch owns RW consecutive weight rows, i.e. RW * rowbytes
//     contiguous bytes; its 64 lanes take consecutive 16-byte pieces of that range
//     (lane i: pieces i, i + 64, ...), so every load instruction of the wavefront covers
//     1 KiB of contiguous memory and the launch walks the matrix in address order;
//   * the workgroup count is chosen so that every CU holds the same number of
//     wavefronts (N = 2560, K = 9728: 256 workgroups of 10 wavefronts, one row each);
//   * every weight and scale load of the wavefront is issued before anything waits, the
//     activation rows are staged in LDS meanwhile (once per workgroup, already permuted
//     into the order in which the codes unpack), and each piece is multiplied as soon as
//     its own load has arrived (loads complete in order).
// A piece is 32 int4 or 16 int8 codes of one row, inside one quantization group. Codes
// become bf16 values (int4: 128 + code, one AND-OR per pair of codes; int8: the signed
// code, one sign-extending byte convert per code), multiplied with v_dot2c_f32_bf16
// against the staged activations in fp32; for int4 the 128 offset is removed with the
// piece's activation sum (staged with the rows). At
// M = 1 the multiply, not the loads, sets the time beyond the streaming read (MI355X,
// N = 2560, K = 9728: 3.7 us with the loads alone, 4.9 us with the multiply alone, 5.6 us
// together), so the address arithmetic is division-free and every wavefront keeps four
// independent dot chains per piece. The MFMA form of the same dot products (each lane
// quad's sum on the diagonal of a 16x16x32 MFMA) issues fewer VALU instructions but
// measured slower (5.95 us): each round waits on a chain of four MFMAs.
//   int4  acc += s_g * (sum x (128 + u) + bias * sum x) [+ z_g * sum x]
//         (bias -136 for symmetric codes, -128 with zero points)
//   int8  y = bf16(bf16(sum x q) * bf16(s))                       (int8_wo.py:17-21)
// The lanes' partial sums of a row are added by a fixed DPP tree, so results are
// deterministic; there is no workspace and no cross-workgroup exchange.
#include <algorithm>
#include <mutex>

#include "wo_core.h"

// Ablation bits for timing probes, compiled in only with -DMIQ_GV_ABL=<bits> (results
// are then wrong): 1 no multiply, 2 no activation staging, 4 no weight loads. The shipped
// library has 0.
#ifndef MIQ_GV_ABL
#define MIQ_GV_ABL 0
#endif

namespace miq {
namespace {

using namespace wo;

constexpr int kGvAbl = MIQ_GV_ABL;
constexpr int kCUs = 256;          // MI355X compute units
constexpr int kGvMaxWaves = 16;    // wavefronts per workgroup at most
constexpr int kGvMaxPieces = 6;    // 16-byte weight pieces per lane (all in flight at once)
constexpr int kGvLds = 150 * 1024; // activation rows + piece sums per workgroup, at most

struct GemvParams {
  const uint16_t* x;
  int64_t ldx;
  const uint8_t* w;
  int64_t ldw;          // bytes per weight row
  const void* scale;
  const void* zero;
  int64_t ngroups;      // scale entries per row (int4); int8: 1
  int group_shift;      // log2 of the pieces per quantization group (int4: group / 32)
  int ldx32, ldw32, ngroups32;  // the strides as 32-bit values (the host checks they fit)
  uint16_t* y;
  int64_t ldy;
  int M, N, K;
  int rows_per_wave;    // RW
  int ppr;              // pieces per weight row
  int wbytes, sbytes, xbytes;
};

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

__device__ inline float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c, false);
}

// 4 signed int8 codes -> 2 dwords of bf16 pairs (exact: |q| <= 128 has at most 8
// significant bits); the byte selects become SDWA sign-extending converts
__device__ inline void s8x4_to_bf16(uint32_t w, uint32_t& lo, uint32_t& hi) {
  const float f0 = (float)(int8_t)(w & 0xff), f1 = (float)(int8_t)((w >> 8) & 0xff);
  const float f2 = (float)(int8_t)((w >> 16) & 0xff), f3 = (float)(int8_t)(w >> 24);
  lo = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, f1), __builtin_bit_cast(uint32_t, f0), 0x07060302u);
  hi = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, f3), __builtin_bit_cast(uint32_t, f2), 0x07060302u);
}

template <int CTRL>
__device__ inline float dpp_add(float v) {
  return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}

// sum over the 64 lanes (uniform result): a DPP tree within each row of 16 lanes, then
// the four row sums in a fixed order (deterministic)
__device__ inline float wave_sum(float v) {
  v = dpp_add<0xB1>(v);   // quad_perm 1,0,3,2
  v = dpp_add<0x4E>(v);   // quad_perm 2,3,0,1
  v = dpp_add<0x124>(v);  // row_ror 4
  v = dpp_add<0x128>(v);  // row_ror 8
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
  return (r0 + r1) + (r2 + r3);
}

constexpr int kGvXPR = 2;  // 16-byte activation pieces per thread and activation row (K / 8 <= 2 * threads)

template <int KIND, bool HZ, int SD, int MR>
__global__ void __launch_bounds__(kGvMaxWaves * 64)
wo_gemv_kernel(GemvParams p) {
  extern __shared__ __align__(16) uint32_t lds32[];
  constexpr bool I4 = KIND == KIND_INT4;
  constexpr int kPieceK = I4 ? 32 : 16;               // k per 16-byte piece
  constexpr int kChunks = kPieceK / 8;                // 8-k chunks per piece
  constexpr float kXBias = HZ ? -128.f : -136.f;      // int4: the dot sees codes as 128 + u
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nthreads = blockDim.x;
  const int M = p.M, K = p.K;
  const int RW = p.rows_per_wave;
  const int row0 = (blockIdx.x * (nthreads >> 6) + wv) * RW;  // first weight row of this wavefront

  // ---- 1. the activation pieces this thread stages (requested first: the staging
  // waits for these only, not for the weight loads issued after them).
  // Out-of-range requests go to an offset past every buffer (the hardware returns zeros
  // and touches no memory); offsets pass through an empty asm so that the compiler keeps
  // one unconditional load per request instead of branching around it. With straight-line
  // loads the compiler's wait before each use counts only the loads issued before it.
  constexpr int kOut = 0x7ffffff0;
  const int p8 = K / 8;  // 16-byte activation pieces per row
  const __amdgpu_buffer_rsrc_t xrs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(p.x), 0, p.xbytes, 0x00020000);
  uint4 xv[MR][kGvXPR];
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int t = 0; t < kGvXPR; ++t) {
      const int c = tid + t * nthreads;
      int off = m < M && c < p8 && !(kGvAbl & 2) ? (m * p.ldx32 + c * 8) * 2 : kOut;
      asm volatile("" : "+v"(off));
      const auto v = __builtin_amdgcn_raw_buffer_load_b128(xrs, off, 0, 0);
      xv[m][t] = *reinterpret_cast<const uint4*>(&v);
    }

  // ---- 2. every weight and scale load of the wavefront: lane l takes pieces l, l + 64,
  // ... of the wavefront's range, so each load instruction covers 1 KiB of contiguous
  // memory
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(p.w), 0, p.wbytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p.scale), 0, p.sbytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t zrs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(HZ ? p.zero : p.scale), 0, p.sbytes, 0x00020000);
  constexpr int esz = SD == MIQ_F32 ? 4 : 2;
  const int npc = K / kPieceK;  // pieces per row
  const int npieces = RW * npc;
  uint4 wq[kGvMaxPieces];
  uint32_t sraw[kGvMaxPieces], zraw[kGvMaxPieces], rsc[2];
  int pslot[kGvMaxPieces], pcol[kGvMaxPieces];
#pragma unroll
  for (int i = 0; i < kGvMaxPieces; ++i) {
    const int j = lane + 64 * i;
    const int rr = j >= npc ? 1 : 0, c = j - rr * npc;  // RW <= 2 rows (host plan): no division
    const int row = row0 + rr;
    const bool ok = j < npieces && row < p.N;
    pslot[i] = rr;
    pcol[i] = c;
    int off = ok ? row * p.ldw32 + c * 16 : kOut;
    asm volatile("" : "+v"(off));
    if constexpr ((kGvAbl & 4) != 0) {  // probe: synthetic weights, no weight loads
      wq[i] = make_uint4(off * 0x9e3779b1u, off ^ 0x5bd1e995u, off + 0x1234567u, off * 3u);
    } else {
      const auto v = __builtin_amdgcn_raw_buffer_load_b128(wrs, off, 0, 2 /* nt: read once */);
      wq[i] = *reinterpret_cast<const uint4*>(&v);
    }
    if constexpr (I4) {
      int soff = ok ? (row * p.ngroups32 + (c >> p.group_shift)) * esz : kOut;
      asm volatile("" : "+v"(soff));
      if constexpr (esz == 4) sraw[i] = __builtin_amdgcn_raw_buffer_load_b32(srs, soff, 0, 0);
      else sraw[i] = __builtin_amdgcn_raw_buffer_load_b16(srs, soff, 0, 0);
      if constexpr (HZ) {
        if constexpr (esz == 4) zraw[i] = __builtin_amdgcn_raw_buffer_load_b32(zrs, soff, 0, 0);
        else zraw[i] = __builtin_amdgcn_raw_buffer_load_b16(zrs, soff, 0, 0);
      }
    }
  }
  if constexpr (!I4) {  // the row scales of the wavefront's (at most two) rows
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
      int soff = rr < RW && row0 + rr < p.N ? (row0 + rr) * esz : kOut;
      asm volatile("" : "+v"(soff));
      if constexpr (esz == 4) rsc[rr] = __builtin_amdgcn_raw_buffer_load_b32(srs, soff, 0, 0);
      else rsc[rr] = __builtin_amdgcn_raw_buffer_load_b16(srs, soff, 0, 0);
    }
  }
  (void)zraw;
  (void)rsc;

  // ---- 3. stage the activation rows in LDS: chunk e (8 k) of piece c at dword
  // m K/2 + (e npc + c) 4, so that the lanes of a wavefront, which take consecutive pieces,
  // read consecutive 16-byte chunks (no bank conflicts); int4 chunks in the unpack order
  // (x0, x4), (x1, x5), (x2, x6), (x3, x7). With them, the activation sum of every piece:
  // each thread sums its 8 values, then the threads of a piece (4 for int4, 2 for int8)
  // add theirs by DPP in a fixed order.
  uint32_t* xl = lds32;                                          // [M][K / 2] dwords
  float* xs = reinterpret_cast<float*>(lds32 + MR * (K / 2));   // [M][npc]
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int t = 0; t < kGvXPR; ++t) {
      const int c8 = tid + t * nthreads;
      const uint4 v = xv[m][t];
      float s8 = 0.f;
      if constexpr (I4) {
        s8 = dot2(v.x, 0x3f803f80u, 0.f);
        s8 = dot2(v.y, 0x3f803f80u, s8);
        s8 = dot2(v.z, 0x3f803f80u, s8);
        s8 = dot2(v.w, 0x3f803f80u, s8);
        s8 = dpp_add<0xB1>(s8);  // pairs of threads (16 k)
        s8 = dpp_add<0x4E>(s8);  // quads (32 k)
      }
      if (m < M && c8 < p8) {
        const int pc = c8 / kChunks, e = c8 - pc * kChunks;
        *reinterpret_cast<uint4*>(xl + m * (K / 2) + (e * npc + pc) * 4) = I4 ? permute_for_u4(v) : v;
        if (I4 && e == 0) xs[m * npc + pc] = s8;
      }
    }
  __syncthreads();

  if constexpr ((kGvAbl & 1) != 0) {  // probe: consume the loads without the multiply
    uint32_t z = 0;
#pragma unroll
    for (int i = 0; i < kGvMaxPieces; ++i) z ^= wq[i].x ^ wq[i].y ^ wq[i].z ^ wq[i].w ^ (I4 ? sraw[i] : 0u);
    if (z == 0x12345678u) p.y[lane] = 0;
    return;
  }

  // ---- 4. the pieces, each as soon as its load has arrived: v_dot2c_f32_bf16 of the
  // unpacked codes against the staged activations, one chain per 32-bit word of codes
  float acc[MR][2];  // per activation row, for the (at most two) weight rows a lane meets
#pragma unroll
  for (int m = 0; m < MR; ++m) acc[m][0] = acc[m][1] = 0.f;
  uint32_t mk, ob;
  asm("" : "=s"(mk) : "0"(0x000f000fu));
  asm("" : "=v"(ob) : "0"(0x43004300u));
#pragma unroll
  for (int i = 0; i < kGvMaxPieces; ++i) {
    if (64 * i >= npieces) break;  // uniform: no lane has piece i
    const uint32_t wd[4] = {wq[i].x, wq[i].y, wq[i].z, wq[i].w};
    const int c = pcol[i];
    const bool live = lane + 64 * i < npieces;
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      if (m >= M) break;
      const uint32_t* xr = xl + m * (K / 2) + c * 4;
      float de[4];  // one chain per word of codes: four independent dot chains
      if constexpr (I4) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint4 xq = *reinterpret_cast<const uint4*>(xr + e * npc * 4);
          const uint32_t w = wd[e];
          de[e] = dot2((w & mk) | ob, xq.x, 0.f);
          de[e] = dot2(((w >> 4) & mk) | ob, xq.y, de[e]);
          de[e] = dot2(((w >> 8) & mk) | ob, xq.z, de[e]);
          de[e] = dot2(((w >> 12) & mk) | ob, xq.w, de[e]);
        }
      } else {
        // int8: the signed codes themselves (no 128 offset, so no activation sums)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint4 xq = *reinterpret_cast<const uint4*>(xr + h * npc * 4);
          uint32_t lo, hi;
          s8x4_to_bf16(wd[2 * h], lo, hi);
          de[h] = dot2(lo, xq.x, 0.f);
          de[h] = dot2(hi, xq.y, de[h]);
          s8x4_to_bf16(wd[2 * h + 1], lo, hi);
          de[h] = dot2(lo, xq.z, de[h]);
          de[h] = dot2(hi, xq.w, de[h]);
        }
        de[2] = de[3] = 0.f;
      }
      const float d = I4 ? (de[0] + de[1]) + (de[2] + de[3]) : de[0] + de[1];
      float t;
      if constexpr (I4) {
        const float xsum = xs[m * npc + c];
        t = sd_to_f32<SD>(sraw[i]) * __builtin_fmaf(kXBias, xsum, d);
        if constexpr (HZ) t = __builtin_fmaf(sd_to_f32<SD>(zraw[i]), xsum, t);
      } else {
        t = d;
      }
      t = live ? t : 0.f;
      acc[m][0] += pslot[i] ? 0.f : t;  // selects, not branches
      acc[m][1] += pslot[i] ? t : 0.f;
    }
  }

  // ---- 5. rows: slot 0 of a lane holds parts of the wavefront's row 0, slot 1 of row 1
#pragma unroll
  for (int rr = 0; rr < 2; ++rr) {
    const int row = row0 + rr;
    if (rr >= RW) break;
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      if (m >= M) break;
      const float tot = wave_sum(acc[m][rr]);
      if (lane == 0 && row < p.N) {
        if constexpr (!I4) {
          const float a = bf16_to_f32(f32_to_bf16(tot));
          const float s = bf16_to_f32(f32_to_bf16(sd_to_f32<SD>(rsc[rr])));
          p.y[(int64_t)m * p.ldy + row] = f32_to_bf16(a * s);
        } else {
          p.y[(int64_t)m * p.ldy + row] = f32_to_bf16(tot);
        }
      }
    }
  }
}

}  // namespace
}  // namespace miq

namespace miq {
namespace {

template <int KIND, bool HZ, int SD, int MR>
void launch_gemv(const GemvParams& p, unsigned grid, unsigned threads, size_t lds, hipStream_t st) {
  static std::once_flag lds_once;  // the LDS limit is raised once per kernel (thread-safe)
  std::call_once(lds_once, [] { allow_max_dynamic_lds(reinterpret_cast<const void*>(&wo_gemv_kernel<KIND, HZ, SD, MR>)); });
  hipLaunchKernelGGL((wo_gemv_kernel<KIND, HZ, SD, MR>), dim3(grid), dim3(threads), lds, st, p);
}

// activation rows of the kernel instance that takes M rows. Instances for 4 and 8 rows
// measured slower than the tile and streamed kernels on MI355X (INT8 N = 19456, K = 2560:
// M = 4 / 8 17.4 / 33.5 against 13.1 / 15.5 us; INT4 N = 2560, K = 9728, M = 4: 7.8 us with
// 8-wavefront workgroups against 8.1), so at most 2 rows are built
constexpr int gemv_rows(int64_t M) { return M <= 1 ? 1 : 2; }

template <int KIND, bool HZ, int SD>
void launch_m(int M, const GemvParams& p, unsigned grid, unsigned threads, size_t lds, hipStream_t st) {
  if (gemv_rows(M) == 1) launch_gemv<KIND, HZ, SD, 1>(p, grid, threads, lds, st);
  else launch_gemv<KIND, HZ, SD, 2>(p, grid, threads, lds, st);
}

}  // namespace

// The GEMV plan: rows per wavefront, wavefronts per workgroup (0: the kernel does not apply).
struct GemvPlan {
  int RW, W, ppr;
  size_t lds_bytes;
};

GemvPlan plan_gemv(int kind, int64_t M, int64_t N, int64_t K) {
  GemvPlan pl{};
  const Tuning& tu = tuning();
  if (tu.wo_stream) return pl;  // MIQ_WO_STREAM forces the streamed kernel
  const int max_m = tu.wo_gemv_max_m >= 0 ? std::min(tu.wo_gemv_max_m, 2) : 1;
  if (M < 1 || M > max_m || N < 1 || K < kStepK) return pl;
  const int64_t piece_k = kind == KIND_INT4 ? 32 : 16;
  const int64_t ppr = K / piece_k;
  int RW = 0;
  for (int rw = 2; rw >= 1 && RW == 0; --rw)
    if ((rw * ppr + 63) / 64 <= kGvMaxPieces) RW = rw;
  if (RW == 0) return pl;
  // int4: about one workgroup per CU (N = 2560, K = 9728 on MI355X: 10 wavefronts, 5.5-5.6
  // us against 6.2-6.3 with 8, 12 or 16); int8: workgroups of 4 wavefronts (N = 19456,
  // K = 2560: 10.6-10.7 us against 10.7-11.1 with 8 and 13.0-13.5 with 16)
  const int64_t waves = (N + RW - 1) / RW;
  int W = kind == KIND_INT8 ? 4 : (int)std::min<int64_t>(kGvMaxWaves, std::max<int64_t>(1, (waves + kCUs - 1) / kCUs));
  if (tu.wo_gemv_waves > 0) W = std::min(tu.wo_gemv_waves, kGvMaxWaves);
  const int64_t threads = 64LL * W;
  if (K / 8 > kGvXPR * threads) return pl;  // activation pieces per thread and row
  const size_t lds = (size_t)gemv_rows(M) * ((size_t)K * 2 + (size_t)ppr * 4);
  if (lds > (size_t)kGvLds) return pl;
  pl.RW = RW;
  pl.W = W;
  pl.ppr = (int)ppr;
  pl.lds_bytes = lds;
  return pl;
}

// Launches the GEMV kernel when it applies (`launched` says whether it did).
int wo_gemv_launch(int kind, const uint16_t* x, int64_t ldx, const uint8_t* w, int64_t ldw, const void* scale,
                   const void* zero, int sd, int group_steps, int64_t ngroups, uint16_t* y, int64_t ldy, int M,
                   int N, int K, hipStream_t st, const char* name, bool& launched) {
  launched = false;
  const GemvPlan pl = plan_gemv(kind, M, N, K);
  if (pl.RW == 0) return MIQ_OK;
  const int gp = group_steps * (kStepK / 32);
  if (kind == KIND_INT4 && (gp & (gp - 1)) != 0) return MIQ_OK;  // groups of a power-of-two piece count only
  MIQ_REQUIRE((int64_t)N * ldw < 0x7fff0000LL, "%s: weights of %lld bytes exceed 2 GiB", name, (long long)N * ldw);
  MIQ_REQUIRE(ldw % 16 == 0, "%s: weight rows must be a multiple of 16 bytes", name);
  MIQ_REQUIRE((int64_t)M * ldx * 2 < 0x7fff0000LL, "%s: activations exceed 2 GiB", name);
  GemvParams p{};
  p.x = x;
  p.ldx = ldx;
  p.w = w;
  p.ldw = ldw;
  p.scale = scale;
  p.zero = zero;
  p.ngroups = ngroups;
  p.group_shift = __builtin_ctz((unsigned)gp);
  p.ldx32 = (int)ldx;
  p.ldw32 = (int)ldw;
  p.ngroups32 = (int)ngroups;
  p.y = y;
  p.ldy = ldy;
  p.M = M;
  p.N = N;
  p.K = K;
  p.rows_per_wave = pl.RW;
  p.ppr = pl.ppr;
  p.wbytes = (int)((int64_t)N * ldw);
  p.xbytes = (int)((int64_t)(M - 1) * ldx * 2 + (int64_t)K * 2);
  const int esz = sd == MIQ_F32 ? 4 : 2;
  p.sbytes = (int)(((int64_t)N * ngroups * esz + 3) & ~3LL);
  const int64_t waves = (N + pl.RW - 1) / pl.RW;
  const unsigned grid = (unsigned)((waves + pl.W - 1) / pl.W);
  const unsigned threads = (unsigned)(64 * pl.W);
  if (kind == KIND_INT8) {
    if (sd == MIQ_BF16) launch_m<KIND_INT8, false, MIQ_BF16>(M, p, grid, threads, pl.lds_bytes, st);
    else if (sd == MIQ_F16) launch_m<KIND_INT8, false, MIQ_F16>(M, p, grid, threads, pl.lds_bytes, st);
    else launch_m<KIND_INT8, false, MIQ_F32>(M, p, grid, threads, pl.lds_bytes, st);
  } else if (zero) {
    if (sd == MIQ_BF16) launch_m<KIND_INT4, true, MIQ_BF16>(M, p, grid, threads, pl.lds_bytes, st);
    else if (sd == MIQ_F16) launch_m<KIND_INT4, true, MIQ_F16>(M, p, grid, threads, pl.lds_bytes, st);
    else launch_m<KIND_INT4, true, MIQ_F32>(M, p, grid, threads, pl.lds_bytes, st);
  } else {
    if (sd == MIQ_BF16) launch_m<KIND_INT4, false, MIQ_BF16>(M, p, grid, threads, pl.lds_bytes, st);
    else if (sd == MIQ_F16) launch_m<KIND_INT4, false, MIQ_F16>(M, p, grid, threads, pl.lds_bytes, st);
    else launch_m<KIND_INT4, false, MIQ_F32>(M, p, grid, threads, pl.lds_bytes, st);
  }
  launched = true;
  return check_launch(name);
}

}  // namespace miq
