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
#include <cstdlib>
#include <type_traits>

#include <mutex>

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
  // the LDS limit is set once per kernel (thread-safe)
  static std::once_flag lds_once;
  std::call_once(lds_once, [&] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&fp8_gemm_kernel<BM, BN, WM, WN>),
                        hipFuncAttributeMaxDynamicSharedMemorySize, (int)C::kLds);
  });
  hipLaunchKernelGGL((fp8_gemm_kernel<BM, BN, WM, WN>), dim3((unsigned)(tm * tn)), dim3(C::kThreads),
                     C::kLds, st, xq, xs, wq, ws, y, ldy, M, N, K, tm, tn, xcd);
  return check_launch("fp8_gemm");
}


// ---------------------------------------------------------------- 32x32 MFMA kernel
// The large-tile kernel: a 256 x 192 tile per workgroup (one per CU at the prefill shape),
// 4 wavefronts of 128 x 96 each on v_mfma_scale_f32_32x32x64_f8f6f4 (12 accumulator
// tiles of 32 x 32 = 192 fp32 per lane, in AGPRs).
//
// Operands go from HBM straight to LDS (buffer_load_dwordx4 ... lds: no registers, no
// LDS store instructions) through a ring of NS stages of 64 k; stage s + NS - 1 is
// requested while stage s is multiplied, so NS - 1 stages of load latency are hidden.
// A stage is 256 + 192 rows of 64 bytes; each wavefront issues 7 of its 28 one-KiB
// loads. One wait on the wavefront's own loads and one barrier per stage.
//
// LDS row layout: the 4 chunks of 16 bytes of row R sit at positions c ^ ((R >> 2) & 3),
// so the 16 rows that 16 lanes read for one fragment hit 16 different 4-bank groups. A
// load writes 64 lanes x 16 bytes contiguously, so each lane fetches the global chunk
// that belongs at its position.
//
// Fragments: for the 32x32x64 MFMA, lane l supplies 32 bytes of row l % 32 of A (and of
// column l % 32 of B) at k offset (l / 32) * 32; A and B use the same offsets, so the
// instruction's internal byte order cannot change the dot product. Accumulator element i
// of lane l is C[row (i / 4) * 8 + (l / 32) * 4 + i % 4][col l % 32].
#ifndef MIQ_FP8_PREFETCH
#define MIQ_FP8_PREFETCH 1
#endif
constexpr int BK32 = 64;                 // k per stage
constexpr int kStages32 = 5;             // ring depth

__device__ inline f32x16 mfma32_fp8(i32x8 a, i32x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

template <int N>
__device__ inline void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

template <int BM, int BN, int WV>
__global__ void __launch_bounds__(WV * 64)
fp8_gemm32_kernel(const uint8_t* __restrict__ A, const float* __restrict__ sa,
                  const uint8_t* __restrict__ B, const float* __restrict__ sb,
                  uint16_t* __restrict__ Y, int64_t ldy, int M, int N, int K, int tiles_m,
                  int tiles_n, int xcd_panels) {
  // WV = 4: 2 x 2 wavefronts of 128 x 96; WV = 8: 4 x 2 of 64 x 96 (two per SIMD)
  constexpr int WM = WV == 8 ? 4 : 2, WN = 2, NS = kStages32;
  constexpr int kWaveM = BM / WM, kWaveN = BN / WN;
  constexpr int kTM = kWaveM / 32, kTN = kWaveN / 32;  // 32 x 32 tiles per wavefront
  constexpr int kRowBytes = BK32;                      // 64
  constexpr int kStage = (BM + BN) * kRowBytes;        // 28 KiB
  constexpr int kLoadsA = BM / 16, kLoadsB = BN / 16;  // 1-KiB loads (16 rows) per stage
  extern __shared__ __align__(16) uint8_t smem[];
  const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wv / WN, wn = wv - wm * WN;

  int tm, tn;
  const int bid = blockIdx.x;
  if (xcd_panels) {  // each XCD walks all row tiles of its band of column tiles (B stays in its L2)
    const int xcd = bid & 7, local = bid >> 3;
    tm = local % tiles_m;
    tn = xcd * (tiles_n / 8) + local / tiles_m;
  } else {
    tm = bid % tiles_m;
    tn = bid / tiles_m;
  }
  const int m0 = tm * BM, n0 = tn * BN;

  // this lane's part of every load: row lane / 4 of the 16, global chunk (lane & 3) ^
  // ((lane >> 4) & 3); rows past M or N read zeros (the descriptor's size)
  const __amdgpu_buffer_rsrc_t ars = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(A), 0, M * K, 0x00020000);
  const __amdgpu_buffer_rsrc_t brs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(B), 0, N * K, 0x00020000);
  const int lrow = lane >> 2, lchunk = (lane & 3) ^ ((lane >> 4) & 3);
  const int voffA = (m0 + lrow) * K + lchunk * 16, voffB = (n0 + lrow) * K + lchunk * 16;
  typedef __attribute__((address_space(3))) void* lds_ptr;
  // WV = 4: wavefront w issues A loads 4 w .. 4 w + 3 and B loads 3 w .. 3 w + 2 of each
  // stage; WV = 8: A loads 2 w, 2 w + 1 and B loads 2 w, 2 w + 1 (w < 4) or 4 + w (w >= 4)
  static_assert(kLoadsA == 16 && kLoadsB == 12, "load split assumes a 256 x 192 tile");
  constexpr int nA = kLoadsA / WV, nBmax = WV == 4 ? 3 : 2;
  const int qa0 = wv * nA;
  const int nB = WV == 4 ? 3 : (wv < 4 ? 2 : 1);
  const int qb0 = WV == 4 ? wv * 3 : (wv < 4 ? wv * 2 : 4 + wv);
  auto issue = [&](int st, int slot) {  // stage st into ring slot `slot`
    uint8_t* base = smem + slot * kStage;
    const int k0 = st * BK32;
#pragma unroll
    for (int u = 0; u < nA; ++u)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ars, (lds_ptr)(base + (qa0 + u) * 1024), 16, voffA + k0,
                                               (qa0 + u) * 16 * K, 0, 0);
#pragma unroll
    for (int u = 0; u < nBmax; ++u)
      if (u < nB)  // uniform
        __builtin_amdgcn_raw_ptr_buffer_load_lds(brs, (lds_ptr)(base + BM * kRowBytes + (qb0 + u) * 1024), 16,
                                                 voffB + k0, (qb0 + u) * 16 * K, 0, 0);
  };

  f32x16 acc[kTM][kTN];
#pragma unroll
  for (int i = 0; i < kTM; ++i)
#pragma unroll
    for (int j = 0; j < kTN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  // fragment of rows row0 + (lane % 32) (row0 a multiple of 32): chunks 2 (lane / 32) and
  // + 1, at positions that depend on the lane only
  const int fr = lane & 31, fq = lane >> 5;
  const int fsw = (fr >> 2) & 3;
  const int foff0 = fr * kRowBytes + (((fq * 2) ^ fsw) << 4), foff1 = fr * kRowBytes + (((fq * 2 + 1) ^ fsw) << 4);
  auto frag = [&](const uint8_t* buf, int row0) -> i32x8 {
    const i32x4 lo = *reinterpret_cast<const i32x4*>(buf + row0 * kRowBytes + foff0);
    const i32x4 hi = *reinterpret_cast<const i32x4*>(buf + row0 * kRowBytes + foff1);
    return i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  };

  // per-wavefront wait for its own loads of the stage N stages back
  auto wait_stage = [&](auto nst_c) {
    constexpr int NSB = decltype(nst_c)::value;  // stages of loads allowed in flight
    if (WV == 4) wait_vmcnt<NSB * 7>();
    else if (wv < 4) wait_vmcnt<NSB * 4>();  // 2 A + 2 B loads per stage
    else wait_vmcnt<NSB * 3>();              // 2 A + 1 B
  };
  const int nsteps = K / BK32;
#pragma unroll
  for (int st = 0; st < NS - 1; ++st)
    if (st < nsteps) issue(st, st);
#if MIQ_FP8_PREFETCH
  // Fragments are read one stage ahead: step s multiplies fragments read from LDS during
  // step s - 1, while the reads of stage s + 1 are in flight. Two register sets, used
  // alternately (the loop is unrolled by 2; nsteps is even since K % 128 == 0). With
  // eight wavefronts this measured 4 % faster on MI355X (38.2 against 39.8 us).
  // MIQ_FP8_PREFETCH=0 builds the loop that reads each stage's fragments when it
  // multiplies them.
  struct Frags {
    i32x8 a[kTM], b[kTN];
  };
  auto read_frags = [&](Frags& f, const uint8_t* buf) {
#pragma unroll
    for (int j = 0; j < kTN; ++j) f.b[j] = frag(buf + BM * kRowBytes, wn * kWaveN + j * 32);
#pragma unroll
    for (int i = 0; i < kTM; ++i) f.a[i] = frag(buf, wm * kWaveM + i * 32);
  };
  if (nsteps >= NS - 1) wait_stage(std::integral_constant<int, NS - 2>{});
  else wait_vmcnt<0>();
  asm volatile("s_barrier" ::: "memory");
  Frags f0, f1;
  int next_slot = 1, free_slot = NS - 1;  // slots of stage s + 1 and of stage s - 1
  auto step = [&](const Frags& fc, Frags& fn, int s) {
    if (s + 1 < nsteps) {
      if (s + NS - 2 < nsteps) wait_stage(std::integral_constant<int, NS - 3>{});
      else wait_vmcnt<0>();
      asm volatile("s_barrier" ::: "memory");
      if (s + NS - 1 < nsteps) issue(s + NS - 1, free_slot);
    }
    // the next stage's fragments are read on every step (after the last one they are read
    // and not used): with the reads on one path only, the compiler's wait before the MFMAs
    // below covered every LDS read in flight, these ones too (MI355X: 39.0 -> 37.9 us at
    // 2048 x 6144 x 2560). Issuing them as inline asm with explicit waits for the step
    // before's reads only measured slower (39.4 us) than the compiler's placement, which
    // interleaves them with the MFMAs.
    read_frags(fn, smem + next_slot * kStage);
    next_slot = next_slot == NS - 1 ? 0 : next_slot + 1;
    free_slot = free_slot == NS - 1 ? 0 : free_slot + 1;
#pragma unroll
    for (int i = 0; i < kTM; ++i)
#pragma unroll
      for (int j = 0; j < kTN; ++j) acc[i][j] = mfma32_fp8(fc.a[i], fc.b[j], acc[i][j]);
  };
  read_frags(f0, smem);
  for (int s = 0; s < nsteps; s += 2) {
    step(f0, f1, s);
    step(f1, f0, s + 1);
  }
#else
  int slot = 0, next_slot = NS - 1;  // ring slots of stage s and of stage s + NS - 1
  for (int s = 0; s < nsteps; ++s) {
    // this wavefront's loads of stage s are done once at most (NS - 2) stages of loads
    // issued after it remain; then every wavefront's (barrier), and the slot of stage
    // s - 1 is free for stage s + NS - 1
    if (s + NS - 2 < nsteps) wait_stage(std::integral_constant<int, NS - 2>{});
    else wait_vmcnt<0>();
    // a bare barrier: __syncthreads() would also wait for every load in flight (the later
    // stages too); the fragment reads of stage s - 1 have completed (their MFMAs waited)
    asm volatile("s_barrier" ::: "memory");
    if (s + NS - 1 < nsteps) issue(s + NS - 1, next_slot);
    const uint8_t* cur = smem + slot * kStage;
    slot = slot == NS - 1 ? 0 : slot + 1;
    next_slot = next_slot == NS - 1 ? 0 : next_slot + 1;
    i32x8 bf[kTN];
#pragma unroll
    for (int j = 0; j < kTN; ++j) bf[j] = frag(cur + BM * kRowBytes, wn * kWaveN + j * 32);
#pragma unroll
    for (int i = 0; i < kTM; ++i) {
      const i32x8 af = frag(cur, wm * kWaveM + i * 32);
#pragma unroll
      for (int j = 0; j < kTN; ++j) acc[i][j] = mfma32_fp8(af, bf[j], acc[i][j]);
    }
  }
#endif

  // epilogue: y = bf16(acc * sa[m] * sb[n]). The wavefront's 128 x 96 bf16 tile goes through LDS (the
  // ring is free once every wavefront is past its last stage) and out as 16-byte row
  // pieces, instead of 192 scattered 2-byte stores per lane.
  const int mw = m0 + wm * kWaveM, nw = n0 + wn * kWaveN;
  float wsn[kTN];
#pragma unroll
  for (int j = 0; j < kTN; ++j) wsn[j] = sb[min(nw + j * 32 + fr, N - 1)];
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  constexpr int kCRow = kWaveN + 8;  // bf16 per LDS row of the wavefront's tile
  uint16_t* ct = reinterpret_cast<uint16_t*>(smem) + wv * (kWaveM * kCRow);
#pragma unroll
  for (int i = 0; i < kTM; ++i) {
#pragma unroll
    for (int e4 = 0; e4 < 4; ++e4) {
      const int r0 = i * 32 + e4 * 8 + fq * 4;  // rows r0 .. r0 + 3 of the wavefront tile
      float xsv[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) xsv[e] = sa[min(mw + r0 + e, M - 1)];
#pragma unroll
      for (int j = 0; j < kTN; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          ct[(r0 + e) * kCRow + j * 32 + fr] = f32_to_bf16(acc[i][j][e4 * 4 + e] * xsv[e] * wsn[j]);
    }
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  constexpr int kPiecesRow = kWaveN / 8;                  // 16-byte pieces per row: 12
  constexpr int kPieces = kWaveM * kPiecesRow / 64;       // per lane: 24
#pragma unroll
  for (int u = 0; u < kPieces; ++u) {
    const int pc = lane + u * 64, row = pc / kPiecesRow, col = (pc - row * kPiecesRow) * 8;
    const int m = mw + row, n = nw + col;
    const uint4 v = *reinterpret_cast<const uint4*>(ct + row * kCRow + col);
    if (m < M && n < N) *reinterpret_cast<uint4*>(Y + (int64_t)m * ldy + n) = v;
  }
}

template <int BM, int BN, int WV>
int launch32w(const uint8_t* xq, const float* xs, const uint8_t* wq, const float* ws, uint16_t* y,
              int64_t ldy, int M, int N, int K, hipStream_t st) {
  const int tm = (M + BM - 1) / BM, tn = (N + BN - 1) / BN;
  const int xcd = (tn % 8 == 0) ? 1 : 0;
  constexpr size_t kLds = (size_t)kStages32 * (BM + BN) * BK32;
  // the LDS limit is set once per kernel (thread-safe)
  static std::once_flag lds_once;
  std::call_once(lds_once, [&] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&fp8_gemm32_kernel<BM, BN, WV>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)kLds);
  });
  hipLaunchKernelGGL((fp8_gemm32_kernel<BM, BN, WV>), dim3((unsigned)(tm * tn)), dim3(WV * 64), kLds, st, xq, xs,
                     wq, ws, y, ldy, M, N, K, tm, tn, xcd);
  return check_launch("fp8_gemm");
}

template <int BM, int BN>
int launch32(const uint8_t* xq, const float* xs, const uint8_t* wq, const float* ws, uint16_t* y,
             int64_t ldy, int M, int N, int K, hipStream_t st) {
  // 8 wavefronts (two per SIMD, 64 x 96 each) measured 9 % faster than 4 of 128 x 96 on
  // MI355X (40 against 44 us at 2048 x 6144 x 2560): one wavefront's barrier and LDS
  // waits overlap the other's MFMAs. MIQ_FP8_WAVES=4 runs the 4-wavefront layout.
  const bool four = tuning().fp8_four_waves;
  if (four) return launch32w<BM, BN, 4>(xq, xs, wq, ws, y, ldy, M, N, K, st);
  return launch32w<BM, BN, 8>(xq, xs, wq, ws, y, ldy, M, N, K, st);
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
  if (M >= 1024 && N % 192 == 0) {
    // the large-tile kernel addresses the operands through buffer descriptors (< 2 GiB)
    // and stores 16-byte pieces of y rows
    if (!tuning().fp8_old && M * K < 0x7fffffffLL && N * K < 0x7fffffffLL && ldy % 8 == 0 &&
        (reinterpret_cast<uintptr_t>(y) & 15) == 0)
      return launch32<256, 192>(xq, x_scale, wq, w_scale, yy, ldy, (int)M, (int)N, (int)K, st);
    return launch<256, 192, 4, 2>(xq, x_scale, wq, w_scale, yy, ldy, (int)M, (int)N, (int)K, st);
  }
  return launch<128, 128, 2, 2>(xq, x_scale, wq, w_scale, yy, ldy, (int)M, (int)N, (int)K, st);
}
