// Weight-only quantized skinny GEMMs (decode, M = 1..64) for gfx950.
//
//   y[m, n] = sum_k x[m, k] * W[n, k],  x bf16 [M, K],  W int8 [N, K] or int4 [N, K/2]
//
// Layout of the work (one workgroup = 4 wavefronts = 64 weight rows):
//   * every wavefront owns 16 consecutive weight rows n; all four share one K range, so
//     the activations of that range are staged once per workgroup in LDS;
//   * the K range of a row block is cut into S splits along grid.y when the row blocks
//     alone cannot fill 256 CUs; the last workgroup to finish a row block adds the S
//     fp32 partials in split order (deterministic) and writes bf16;
//   * weights stream from HBM with 16-byte loads: lane (r = lane % 16, g = lane / 16)
//     reads 16 bytes of row n0 + r, so each load instruction moves 1 KiB and one row
//     gets 64 contiguous bytes;
//   * the products run on v_mfma_f32_16x16x32_bf16 with x as the A operand (16 rows of
//     m) and the unpacked weights as the B operand (16 columns of n).
//
// Unpacking without per-element scale work: a 4-bit code u becomes the bf16 value
// 128 + u with one AND-OR (0x4300 | u is exactly 128 + u), and an int8 code q becomes
// 128 + q via an xor and a byte-to-float convert. The MFMA then yields
// sum x * (128 + u); an extra MFMA against a B operand of ones yields sum x, and
//   sum x * q_true = sum x * (128 + u) - 128 * sum x          (exact in fp32 up to rounding)
// so per-group scale / zero (int4) and per-row scale (int8) are applied once per
// 16x16 accumulator tile instead of once per weight.
#include "wo_core.h"

namespace miq {
namespace {

using namespace wo;

constexpr int kThreads = 256;
constexpr int kRowsPerBlock = 64;
constexpr int64_t kMaxCounters = 4096;  // row blocks that may use split-K

struct WoParams {
  const uint16_t* x;
  int64_t ldx;
  const uint8_t* w;
  int64_t ldw;  // bytes per weight row
  const void* scale;
  const void* zero;
  int sz_dtype;
  int group_steps;  // int4: k-steps per quantization group
  int64_t ngroups;  // int4: groups per row (row stride of scale / zero)
  uint16_t* y;
  int64_t ldy;
  int M, N, K;
  int S;           // K splits
  int units;       // K units to split: k-steps (int8) or groups (int4)
  int unit_steps;  // k-steps per unit
  int chunk_steps; // k-steps of x staged in LDS at once
  float* partial;  // [S][M][N]
  int* counters;   // [N / 64]
};

template <int KIND>
__device__ inline void stage_x(const WoParams& p, uint16_t* lds, int lds_stride, int k_step0, int nsteps) {
  const int pieces_per_row = nsteps * (kStepK / 8);
  const int total = p.M * pieces_per_row;
  for (int i = threadIdx.x; i < total; i += kThreads) {
    const int m = i / pieces_per_row, c = i - m * pieces_per_row;
    uint4 v = *reinterpret_cast<const uint4*>(p.x + m * p.ldx + (int64_t)k_step0 * kStepK + c * 8);
    if (KIND == KIND_INT4) v = permute_for_u4(v);
    *reinterpret_cast<uint4*>(lds + m * lds_stride + c * 8) = v;
  }
}

template <int KIND, int MT, bool HAS_ZERO>
__global__ void __launch_bounds__(kThreads)
wo_gemm_kernel(WoParams p) {
  extern __shared__ __align__(16) uint16_t lds_x[];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int n_wave = blockIdx.x * kRowsPerBlock + wv * 16;
  const bool active = n_wave < p.N;
  const int n = n_wave + r;  // weight row of this lane's B data, output column of its C data

  // K range of this split, in whole units
  const int s = blockIdx.y;
  const int u0 = (int)((int64_t)p.units * s / p.S), u1 = (int)((int64_t)p.units * (s + 1) / p.S);
  const int st0 = u0 * p.unit_steps, st1 = u1 * p.unit_steps;

  Acc<MT> st;
  st.clear();
  GroupScales gs{p.scale, p.zero, p.sz_dtype, p.group_steps, (int64_t)(active ? n : 0) * p.ngroups};
  const int lds_stride = p.chunk_steps * kStepK + 8;
  const uint8_t* wrow = p.w + (int64_t)(active ? n : 0) * p.ldw;

  for (int c0 = st0; c0 < st1; c0 += p.chunk_steps) {
    const int nsteps = min(p.chunk_steps, st1 - c0);
    __syncthreads();  // previous chunk fully consumed
    stage_x<KIND>(p, lds_x, lds_stride, c0, nsteps);
    __syncthreads();
    if (active) run_steps<KIND, MT, HAS_ZERO>(wrow, lds_x, lds_stride, p.M, c0, nsteps, r, g, gs, st);
  }
  if (KIND == KIND_INT8) finish_int8<MT>(st);

  // this split's result for rows m = 16 t + 4 g + v, column n
  if (p.S == 1) {
    if (!active) return;
    float ysc = 1.f;
    if (KIND == KIND_INT8) ysc = bf16_to_f32(f32_to_bf16(load_scalar(p.scale, p.sz_dtype, n)));
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int m = t * 16 + g * 4 + v;
        if (m < p.M) {
          float o = st.acc[t][v];
          if (KIND == KIND_INT8) o = bf16_to_f32(f32_to_bf16(o)) * ysc;
          p.y[(int64_t)m * p.ldy + n] = f32_to_bf16(o);
        }
      }
    return;
  }

  // split-K: publish the partial, the last workgroup of this row block reduces
  if (active) {
    float* part = p.partial + (int64_t)s * p.M * p.N;
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int m = t * 16 + g * 4 + v;
        if (m < p.M) part[(int64_t)m * p.N + n] = st.acc[t][v];
      }
  }
  __threadfence();
  __syncthreads();
  __shared__ int s_last;
  if (tid == 0) s_last = atomicAdd(&p.counters[blockIdx.x], 1) == p.S - 1;
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  const int nb = blockIdx.x * kRowsPerBlock;
  const int cols = min(kRowsPerBlock, p.N - nb);
  for (int i = tid; i < p.M * kRowsPerBlock; i += kThreads) {
    const int m = i / kRowsPerBlock, c = i - m * kRowsPerBlock;
    if (c >= cols) continue;
    const int64_t off = (int64_t)m * p.N + nb + c;
    float o = 0.f;
    for (int ss = 0; ss < p.S; ++ss) o += __builtin_nontemporal_load(p.partial + (int64_t)ss * p.M * p.N + off);
    if (KIND == KIND_INT8) {
      const float ysc = bf16_to_f32(f32_to_bf16(load_scalar(p.scale, p.sz_dtype, nb + c)));
      o = bf16_to_f32(f32_to_bf16(o)) * ysc;
    }
    p.y[(int64_t)m * p.ldy + nb + c] = f32_to_bf16(o);
  }
  if (tid == 0) p.counters[blockIdx.x] = 0;
}

// ------------------------------------------------------------------ host-side planning
struct Plan {
  int S, units, unit_steps, chunk_steps;
  size_t lds_bytes, counter_bytes, partial_bytes;
};

Plan make_plan(int64_t M, int64_t N, int64_t K, int weight_bits, int64_t group) {
  Plan pl;
  const int64_t steps = K / kStepK;
  pl.unit_steps = weight_bits == 4 ? (int)(group / kStepK) : 1;
  pl.units = (int)(steps / pl.unit_steps);
  const int64_t nblk = (N + kRowsPerBlock - 1) / kRowsPerBlock;
  // enough workgroups for ~3 per CU, but keep the fp32 partial traffic (written and read
  // once per split) below half of the weight bytes
  int64_t want = (768 + nblk - 1) / nblk;
  const int64_t wbytes_per_row = K * weight_bits / 8;
  int64_t cap = wbytes_per_row / (16 * M);
  if (cap < 1) cap = 1;
  int64_t S = want < cap ? want : cap;
  if (S > pl.units) S = pl.units;
  if (S < 1) S = 1;
  if (nblk > kMaxCounters) S = 1;
  pl.S = (int)S;
  // x chunk in LDS: at most 32 KiB
  int64_t cs = 128 / M;
  if (cs < 1) cs = 1;
  const int64_t max_split_steps = ((pl.units + S - 1) / S) * pl.unit_steps;
  if (cs > max_split_steps) cs = max_split_steps;
  pl.chunk_steps = (int)cs;
  pl.lds_bytes = (size_t)M * (cs * kStepK + 8) * 2;
  // counters live in a fixed region so that partials of a call with another shape
  // never overlap the counters of this one
  pl.counter_bytes = kMaxCounters * 4;
  pl.partial_bytes = S > 1 ? (size_t)S * M * N * 4 : 0;
  return pl;
}

template <int KIND, int MT, bool HZ>
void launch_mt(const WoParams& p, dim3 grid, size_t lds, hipStream_t st) {
  hipLaunchKernelGGL((wo_gemm_kernel<KIND, MT, HZ>), grid, dim3(kThreads), lds, st, p);
}

template <int KIND, bool HZ>
void launch(const WoParams& p, dim3 grid, size_t lds, hipStream_t st) {
  const int mt = (p.M + 15) / 16;
  switch (mt) {
    case 1: launch_mt<KIND, 1, HZ>(p, grid, lds, st); break;
    case 2: launch_mt<KIND, 2, HZ>(p, grid, lds, st); break;
    case 3: launch_mt<KIND, 3, HZ>(p, grid, lds, st); break;
    default: launch_mt<KIND, 4, HZ>(p, grid, lds, st); break;
  }
}

int run(int kind, WoParams p, int64_t group, void* workspace, size_t ws_bytes, hipStream_t st,
        const char* name) {
  MIQ_REQUIRE(p.M >= 1 && p.M <= 64, "%s: M=%d must be in [1, 64]", name, p.M);
  MIQ_REQUIRE(p.K % kStepK == 0 && p.K > 0, "%s: K=%d must be a multiple of 128", name, p.K);
  MIQ_REQUIRE(p.N % 16 == 0 && p.N > 0, "%s: N=%d must be a multiple of 16", name, p.N);
  MIQ_REQUIRE(p.ldx % 8 == 0 && (reinterpret_cast<uintptr_t>(p.x) & 15) == 0,
              "%s: x must be 16-byte aligned with a row stride multiple of 8", name);
  MIQ_REQUIRE((reinterpret_cast<uintptr_t>(p.w) & 15) == 0, "%s: weights must be 16-byte aligned", name);
  MIQ_REQUIRE(p.ldx >= p.K && p.ldy >= p.N, "%s: bad strides", name);
  const Plan pl = make_plan(p.M, p.N, p.K, kind == KIND_INT4 ? 4 : 8, group);
  const size_t need = pl.counter_bytes + pl.partial_bytes;
  if (pl.S > 1) {
    MIQ_REQUIRE(workspace != nullptr && ws_bytes >= need,
                "%s: workspace of %zu bytes needed (got %zu)", name, need, ws_bytes);
  }
  p.S = pl.S;
  p.units = pl.units;
  p.unit_steps = pl.unit_steps;
  p.chunk_steps = pl.chunk_steps;
  p.counters = static_cast<int*>(workspace);
  p.partial = reinterpret_cast<float*>(static_cast<char*>(workspace) + pl.counter_bytes);
  const dim3 grid((unsigned)((p.N + kRowsPerBlock - 1) / kRowsPerBlock), (unsigned)pl.S);
  if (kind == KIND_INT8) launch<KIND_INT8, false>(p, grid, pl.lds_bytes, st);
  else if (p.zero) launch<KIND_INT4, true>(p, grid, pl.lds_bytes, st);
  else launch<KIND_INT4, false>(p, grid, pl.lds_bytes, st);
  return check_launch(name);
}

}  // namespace
}  // namespace miq

using namespace miq;

extern "C" size_t miq_wo_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, int weight_bits) {
  if (M < 1 || N < 1 || K < kStepK) return 256;
  const Plan pl = make_plan(M, N, K, weight_bits, weight_bits == 4 ? kStepK : 0);
  // int4 plans with larger groups never split more finely than group-128 plans
  return pl.counter_bytes + pl.partial_bytes;
}

extern "C" int miq_w8a16_gemm(const void* x, int64_t ldx, const int8_t* q, const void* scale,
                              int scale_dtype, void* y, int64_t ldy, int64_t M, int64_t N, int64_t K,
                              void* workspace, size_t workspace_bytes, void* stream) {
  MIQ_REQUIRE(scale_dtype == MIQ_F32 || scale_dtype == MIQ_BF16 || scale_dtype == MIQ_F16,
              "w8a16_gemm: bad scale dtype");
  MIQ_REQUIRE(N < (1LL << 30) && K < (1LL << 30), "w8a16_gemm: dims too large");
  WoParams p{};
  p.x = static_cast<const uint16_t*>(x);
  p.ldx = ldx;
  p.w = reinterpret_cast<const uint8_t*>(q);
  p.ldw = K;
  p.scale = scale;
  p.zero = nullptr;
  p.sz_dtype = scale_dtype;
  p.group_steps = 1;
  p.ngroups = 1;
  p.y = static_cast<uint16_t*>(y);
  p.ldy = ldy;
  p.M = (int)M;
  p.N = (int)N;
  p.K = (int)K;
  return run(KIND_INT8, p, 0, workspace, workspace_bytes, (hipStream_t)stream, "w8a16_gemm");
}

extern "C" int miq_w4a16_gemm(const void* x, int64_t ldx, const uint8_t* q, const void* scale,
                              const void* zero, int sz_dtype, int64_t group, void* y, int64_t ldy,
                              int64_t M, int64_t N, int64_t K, void* workspace, size_t workspace_bytes,
                              void* stream) {
  MIQ_REQUIRE(sz_dtype == MIQ_F32 || sz_dtype == MIQ_BF16 || sz_dtype == MIQ_F16,
              "w4a16_gemm: bad scale dtype");
  MIQ_REQUIRE(group >= kStepK && group % kStepK == 0 && K % group == 0,
              "w4a16_gemm: group=%lld must be a multiple of 128 dividing K=%lld", (long long)group,
              (long long)K);
  MIQ_REQUIRE(N < (1LL << 30) && K < (1LL << 30), "w4a16_gemm: dims too large");
  WoParams p{};
  p.x = static_cast<const uint16_t*>(x);
  p.ldx = ldx;
  p.w = q;
  p.ldw = K / 2;
  p.scale = scale;
  p.zero = zero;
  p.sz_dtype = sz_dtype;
  p.group_steps = (int)(group / kStepK);
  p.ngroups = K / group;
  p.y = static_cast<uint16_t*>(y);
  p.ldy = ldy;
  p.M = (int)M;
  p.N = (int)N;
  p.K = (int)K;
  return run(KIND_INT4, p, group, workspace, workspace_bytes, (hipStream_t)stream, "w4a16_gemm");
}
