// FP8 (e4m3fn) x FP8 -> bf16 GEMM with per-row and per-column fp32 scales, for gfx950:
//   y[m, n] = bf16( (sum_k xq[m,k] * wq[n,k]) * x_scale[m] * w_scale[n] )
// Both operands are K-contiguous ("TN"), as FP8WeightAct stores them.
//
// One workgroup computes a BM x BN tile with v_mfma_f32_16x16x128_f8f6f4. The K loop
// moves 128 k per step through LDS, double buffered: global loads of step s+1 are issued
// into registers before the MFMAs of step s and written to the other LDS buffer after
// them, so one barrier per step suffices. LDS rows are padded by 16 bytes so that the
// 16 lanes reading 16 different rows hit different banks.
//
// Operand fragments: for the 16x16x128 MFMA each lane supplies 32 bytes of one row of A
// (lane % 16 = row) and of one column of B (lane % 16 = column). Both operands are read
// with the same (lane / 16) * 32 byte offset along k, so whatever order the hardware
// assigns to those 32 bytes inside the instruction, A and B agree and the sum over k is
// the dot product.
#include "miq_common.h"

namespace miq {
namespace {

constexpr int BK = 128;
constexpr int LDS_ROW = BK + 16;

template <int BM, int BN, int WM, int WN>
struct Fp8Cfg {
  static constexpr int kWaves = WM * WN;
  static constexpr int kThreads = kWaves * 64;
  static constexpr int kWaveM = BM / WM;  // rows per wave
  static constexpr int kWaveN = BN / WN;  // cols per wave
  static constexpr int kTM = kWaveM / 16;
  static constexpr int kTN = kWaveN / 16;
  static constexpr int kPieces = (BM + BN) * (BK / 16);  // 16-byte pieces per step
  static constexpr int kLoads = (kPieces + kThreads - 1) / kThreads;
  static constexpr size_t kLds = (size_t)2 * (BM + BN) * LDS_ROW;
};

__device__ inline f32x4 mfma_fp8(i32x8 a, i32x8 b, f32x4 c) {
  // cbsz = blgp = 0: both operands e4m3; scale operands 0 select the unscaled instruction
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

template <int BM, int BN, int WM, int WN>
__global__ void __launch_bounds__(WM * WN * 64)
fp8_gemm_kernel(const uint8_t* __restrict__ A, const float* __restrict__ sa,
                const uint8_t* __restrict__ B, const float* __restrict__ sb,
                uint16_t* __restrict__ Y, int64_t ldy, int M, int N, int K, int tiles_m,
                int tiles_n, int xcd_panels) {
  using C = Fp8Cfg<BM, BN, WM, WN>;
  extern __shared__ __align__(16) uint8_t smem[];
  const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wv / WN, wn = wv - wm * WN;

  // Tile order: consecutive workgroups go to different XCDs (round robin), so give each
  // XCD a band of column tiles and let it walk all row tiles of that band; the band's
  // B panel then stays in that XCD's L2 while A is shared through the MALL.
  int tm, tn;
  const int bid = blockIdx.x;
  if (xcd_panels) {
    const int xcd = bid & 7, local = bid >> 3;
    const int per_xcd_n = tiles_n / 8;
    tm = local % tiles_m;
    tn = xcd * per_xcd_n + local / tiles_m;
  } else {
    tm = bid % tiles_m;
    tn = bid / tiles_m;
  }
  const int m0 = tm * BM, n0 = tn * BN;

  // global -> register staging: each thread moves kLoadsA 16-byte pieces of the A tile and
  // kLoadsB of the B tile per k-step (the configurations divide exactly, so no guards and
  // every array index is a compile-time constant after unrolling)
  static_assert((BM * 8) % C::kThreads == 0 && (BN * 8) % C::kThreads == 0, "tile / thread mismatch");
  constexpr int kLoadsA = BM * 8 / C::kThreads, kLoadsB = BN * 8 / C::kThreads;
  const int c16 = (tid & 7) * 16;
  const int row_step = C::kThreads / 8;
  const uint8_t* srcA = A + (int64_t)min(m0 + (tid >> 3), M - 1) * K + c16;
  const uint8_t* srcB = B + (int64_t)min(n0 + (tid >> 3), N - 1) * K + c16;
  int64_t offA[kLoadsA], offB[kLoadsB];
#pragma unroll
  for (int j = 0; j < kLoadsA; ++j)
    offA[j] = (int64_t)(min(m0 + (tid >> 3) + j * row_step, M - 1) - min(m0 + (tid >> 3), M - 1)) * K;
#pragma unroll
  for (int j = 0; j < kLoadsB; ++j)
    offB[j] = (int64_t)(min(n0 + (tid >> 3) + j * row_step, N - 1) - min(n0 + (tid >> 3), N - 1)) * K;
  const int dst0 = (tid >> 3) * LDS_ROW + c16;
  uint4 ra[kLoadsA], rb[kLoadsB];

  f32x4 acc[C::kTM][C::kTN];
#pragma unroll
  for (int i = 0; i < C::kTM; ++i)
#pragma unroll
    for (int j = 0; j < C::kTN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nsteps = K / BK;
  // prologue: step 0 -> buffer 0
#pragma unroll
  for (int j = 0; j < kLoadsA; ++j) ra[j] = *reinterpret_cast<const uint4*>(srcA + offA[j]);
#pragma unroll
  for (int j = 0; j < kLoadsB; ++j) rb[j] = *reinterpret_cast<const uint4*>(srcB + offB[j]);
#pragma unroll
  for (int j = 0; j < kLoadsA; ++j) *reinterpret_cast<uint4*>(smem + dst0 + j * row_step * LDS_ROW) = ra[j];
#pragma unroll
  for (int j = 0; j < kLoadsB; ++j) *reinterpret_cast<uint4*>(smem + (BM + j * row_step) * LDS_ROW + dst0) = rb[j];
  __syncthreads();

  const int fr = lane & 15, fk = (lane >> 4) * 32;
  for (int s = 0; s < nsteps; ++s) {
    uint8_t* cur = smem + (s & 1) * (BM + BN) * LDS_ROW;
    uint8_t* nxt = smem + ((s + 1) & 1) * (BM + BN) * LDS_ROW;
    const bool more = s + 1 < nsteps;
    const int64_t kn = (int64_t)(more ? s + 1 : s) * BK;  // the last step re-reads (unused)
#pragma unroll
    for (int j = 0; j < kLoadsA; ++j) ra[j] = *reinterpret_cast<const uint4*>(srcA + offA[j] + kn);
#pragma unroll
    for (int j = 0; j < kLoadsB; ++j) rb[j] = *reinterpret_cast<const uint4*>(srcB + offB[j] + kn);
    i32x8 bfr[C::kTN];
#pragma unroll
    for (int j = 0; j < C::kTN; ++j) {
      const uint8_t* p = cur + (BM + wn * C::kWaveN + j * 16 + fr) * LDS_ROW + fk;
      const i32x4 lo = *reinterpret_cast<const i32x4*>(p);
      const i32x4 hi = *reinterpret_cast<const i32x4*>(p + 16);
      bfr[j] = i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
#pragma unroll
    for (int i = 0; i < C::kTM; ++i) {
      const uint8_t* p = cur + (wm * C::kWaveM + i * 16 + fr) * LDS_ROW + fk;
      const i32x4 lo = *reinterpret_cast<const i32x4*>(p);
      const i32x4 hi = *reinterpret_cast<const i32x4*>(p + 16);
      const i32x8 afr = i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
#pragma unroll
      for (int j = 0; j < C::kTN; ++j) acc[i][j] = mfma_fp8(afr, bfr[j], acc[i][j]);
    }
    if (more) {
#pragma unroll
      for (int j = 0; j < kLoadsA; ++j) *reinterpret_cast<uint4*>(nxt + dst0 + j * row_step * LDS_ROW) = ra[j];
#pragma unroll
      for (int j = 0; j < kLoadsB; ++j) *reinterpret_cast<uint4*>(nxt + (BM + j * row_step) * LDS_ROW + dst0) = rb[j];
    }
    __syncthreads();
  }

  // epilogue: lane holds C[row = 4 * (lane / 16) + v][col = lane % 16] of each 16x16 tile
  const int col_l = lane & 15, row_l = (lane >> 4) * 4;
#pragma unroll
  for (int j = 0; j < C::kTN; ++j) {
    const int n = n0 + wn * C::kWaveN + j * 16 + col_l;
    if (n >= N) continue;
    const float wsn = sb[n];
#pragma unroll
    for (int i = 0; i < C::kTM; ++i) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int m = m0 + wm * C::kWaveM + i * 16 + row_l + v;
        if (m < M) Y[(int64_t)m * ldy + n] = f32_to_bf16(acc[i][j][v] * sa[m] * wsn);
      }
    }
  }
}

template <int BM, int BN, int WM, int WN>
int launch(const uint8_t* xq, const float* xs, const uint8_t* wq, const float* ws, uint16_t* y,
           int64_t ldy, int M, int N, int K, hipStream_t st) {
  using C = Fp8Cfg<BM, BN, WM, WN>;
  const int tm = (M + BM - 1) / BM, tn = (N + BN - 1) / BN;
  const int xcd = (tn % 8 == 0) ? 1 : 0;
  static bool attr_set = false;
  if (!attr_set) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&fp8_gemm_kernel<BM, BN, WM, WN>),
                        hipFuncAttributeMaxDynamicSharedMemorySize, (int)C::kLds);
    attr_set = true;
  }
  hipLaunchKernelGGL((fp8_gemm_kernel<BM, BN, WM, WN>), dim3((unsigned)(tm * tn)), dim3(C::kThreads),
                     C::kLds, st, xq, xs, wq, ws, y, ldy, M, N, K, tm, tn, xcd);
  return check_launch("fp8_gemm");
}

}  // namespace
}  // namespace miq

using namespace miq;

extern "C" int miq_fp8_gemm(const uint8_t* xq, const float* x_scale, const uint8_t* wq,
                            const float* w_scale, void* y, int64_t ldy, int64_t M, int64_t N, int64_t K,
                            void* stream) {
  MIQ_REQUIRE(M >= 1 && N >= 1 && K >= BK && K % BK == 0, "fp8_gemm: K=%lld must be a multiple of 128",
              (long long)K);
  MIQ_REQUIRE(M < (1LL << 31) / 2 && N < (1LL << 31) / 2 && K < (1LL << 30), "fp8_gemm: dims too large");
  MIQ_REQUIRE(ldy >= N, "fp8_gemm: ldy < N");
  MIQ_REQUIRE(((reinterpret_cast<uintptr_t>(xq) | reinterpret_cast<uintptr_t>(wq)) & 15) == 0,
              "fp8_gemm: operands must be 16-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  uint16_t* yy = static_cast<uint16_t*>(y);
  if (M >= 1024 && N % 192 == 0)
    return launch<256, 192, 4, 2>(xq, x_scale, wq, w_scale, yy, ldy, (int)M, (int)N, (int)K, st);
  return launch<128, 128, 2, 2>(xq, x_scale, wq, w_scale, yy, ldy, (int)M, (int)N, (int)K, st);
}
