// Weight-only quantized skinny GEMMs (decode, M = 1..64) for gfx950.
//
//   y[m, n] = sum_k x[m, k] * W[n, k],  x bf16 [M, K],  W int8 [N, K] or int4 [N, K/2]
//
// Layout of the work:
//   * a workgroup owns NT tiles of 16 weight rows and a K range (one of S splits along
//     grid.y); its WK wavefronts cut that range into contiguous k slices, stream their
//     slice of all NT tiles and add their 16x16 accumulators in LDS at the end, so no
//     two workgroups share an output unless S > 1;
//   * the activations of the K range are staged in LDS once (all loads issued before
//     the first wait); A fragments come from LDS and are reused by the NT tiles;
//   * weights stream from HBM with 16-byte non-temporal loads, software pipelined: the
//     next batch of k-steps (and the int4 group scales they need) is in flight while the
//     current batch is unpacked and multiplied;
//   * with S > 1 the workgroups of a row block publish fp32 partials with agent-coherent
//     (sc1) stores, wait for them to complete and bump an arrival counter; the last one
//     adds the S partials in split order (deterministic), writes bf16 and resets the
//     counter. No L2 writeback fence is involved.
//
// Unpacking without per-element scale work: a 4-bit code u becomes the bf16 value
// 128 + u with one AND-OR (0x4300 | u is exactly 128 + u), and an int8 code q becomes
// 128 + q via an xor and a byte-to-float convert. The MFMA then yields
// sum x * (128 + u); an extra MFMA against a B operand of ones yields sum x, and
//   sum x * q_true = sum x * (128 + u) - 128 * sum x          (exact in fp32 up to rounding)
// so per-group scale / zero (int4) and per-row scale (int8) are applied once per
// 16x16 accumulator tile instead of once per weight.
#include <stdlib.h>

#include "wo_core.h"

namespace miq {

int wo_decode_launch(int kind, const uint16_t* x, int64_t ldx, const uint8_t* w, int64_t ldw, const void* scale,
                     const void* zero, int sd, int group_steps, int64_t ngroups, uint16_t* y, int64_t ldy, int M, int N,
                     int K, void* workspace, size_t ws_bytes, size_t counter_bytes, hipStream_t st);

namespace {

using namespace wo;

constexpr int kMaxWaves = 8;
constexpr int64_t kMaxCounters = 4096;  // row blocks that may use split-K
constexpr int kLdsBudget = 64 * 1024;   // x chunk staged in LDS

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
  int S;            // K splits over grid.y
  int units;        // K units to split: k-steps (int8) or groups (int4)
  int unit_steps;   // k-steps per unit
  int chunk_steps;  // k-steps of x staged in LDS at once
  float* partial;   // [S][M][N]
  int* counters;    // [kMaxCounters]
};

// Write staged activation pieces (16 bytes = 8 k) to LDS rows; int4 stores them in the
// (0,4,1,5,2,6,3,7) operand order.
template <int KIND>
__device__ inline void commit_x(const Staged<uint4, 8>& st, uint16_t* lds, int lds_stride, int xcols, int first) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    if (j < st.n) {
      const int i = first + threadIdx.x + j * blockDim.x;
      const int m = i / xcols, c = i - m * xcols;
      *reinterpret_cast<uint4*>(lds + m * lds_stride + c * 8) = KIND == KIND_INT4 ? permute_for_u4(st.v[j]) : st.v[j];
    }
  }
}

template <int KIND, int MT, int NT, bool HZ, int SD>
__global__ void __launch_bounds__(kMaxWaves * 64)
wo_gemm_kernel(WoParams p) {
  extern __shared__ __align__(16) uint16_t lds_x[];
  const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6), WK = blockDim.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * 16 * NT;

  const uint8_t* wrow[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int64_t n = n0 + 16 * t < p.N ? n0 + 16 * t + r : 0;
    wrow[t] = p.w + n * p.ldw;
  }

  // K range of this split, in whole units (k-steps for int8, groups for int4)
  const int s = blockIdx.y;
  const int u0 = (int)((int64_t)p.units * s / p.S), u1 = (int)((int64_t)p.units * (s + 1) / p.S);
  const int st0 = u0 * p.unit_steps, st1 = u1 * p.unit_steps;

  f32x4 acc[NT][MT], accg[NT][MT];
  const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) { acc[t][mt] = z4; accg[t][mt] = z4; }

  // LDS: [x chunk][x sums: int4 per group, int8 one per row][int4 scales][int4 zeros]
  const int lds_stride = p.chunk_steps * kStepK + 8;
  constexpr int XR = 16 * MT;
  const int ng = KIND == KIND_INT4 ? u1 - u0 : 0;
  float* xsum = reinterpret_cast<float*>(lds_x + ((p.M * lds_stride + 7) & ~7));
  const int nxs = (KIND == KIND_INT4 ? ng : 1) * XR;
  typedef typename GroupQ<SD>::raw_t raw_t;
  raw_t* lsc = reinterpret_cast<raw_t*>(xsum + nxs);
  const int rows = 16 * NT;
  raw_t* lzr = lsc + rows * ng;
  const GroupQ<SD> q{lsc, HZ ? lzr : nullptr, ng, u0, p.group_steps, xsum, XR};
  for (int i = tid; i < nxs; i += blockDim.x) xsum[i] = 0.f;

  for (int c0 = st0; c0 < st1; c0 += p.chunk_steps) {
    const int c1 = min(c0 + p.chunk_steps, st1);
    // this wave's contiguous slice of the chunk, in whole units
    const int cu0 = c0 / p.unit_steps, cu1 = c1 / p.unit_steps;
    const int a = (cu0 + (int)((int64_t)(cu1 - cu0) * wv / WK)) * p.unit_steps;
    const int b = (cu0 + (int)((int64_t)(cu1 - cu0) * (wv + 1) / WK)) * p.unit_steps;
    if (c0 != st0) __syncthreads();
    // one memory round trip: the first round of x pieces and the group scales are issued,
    // then the weight batch, and only the x / scales are waited for before the LDS writes
    const int xcols = (c1 - c0) * (kStepK / 8);  // 16-byte pieces per activation row
    const uint4* xsrc = reinterpret_cast<const uint4*>(p.x + (int64_t)c0 * kStepK);
    const int xld = (int)(p.ldx / 8);
    Staged<uint4, 8> xs0;
    stage_issue(xs0, xsrc, xld, p.M, xcols, 0);
    const bool do_groups = KIND == KIND_INT4 && c0 == st0;
    const int nrows = min(rows, p.N - n0);
    Staged<raw_t, 4> sg, zg;
    if (do_groups) {
      stage_issue(sg, static_cast<const raw_t*>(p.scale) + (int64_t)n0 * p.ngroups + u0, p.ngroups, nrows, ng, 0);
      if (HZ) stage_issue(zg, static_cast<const raw_t*>(p.zero) + (int64_t)n0 * p.ngroups + u0, p.ngroups, nrows, ng, 0);
    }
    Batch<KIND, NT, 8> ba;  // 8 KiB batches, double buffered
    if (a < b) load_batch<KIND, NT, 8>(wrow, ba, a, b, g);
    commit_x<KIND>(xs0, lds_x, lds_stride, xcols, 0);
    for (int first = 8 * blockDim.x; first < p.M * xcols; first += 8 * blockDim.x) {
      Staged<uint4, 8> more;
      stage_issue(more, xsrc, xld, p.M, xcols, first);
      commit_x<KIND>(more, lds_x, lds_stride, xcols, first);
    }
    if (do_groups) {
      for (int first = 0; first < nrows * ng; first += 4 * blockDim.x) {
        if (first) {
          stage_issue(sg, static_cast<const raw_t*>(p.scale) + (int64_t)n0 * p.ngroups + u0, p.ngroups, nrows, ng, first);
          if (HZ) stage_issue(zg, static_cast<const raw_t*>(p.zero) + (int64_t)n0 * p.ngroups + u0, p.ngroups, nrows, ng, first);
        }
        stage_commit(sg, lsc, ng, nrows, ng, first);
        if (HZ) stage_commit(zg, lzr, ng, nrows, ng, first);
      }
    }
    __syncthreads();
    sum_activations(lds_x, lds_stride, p.M, c1 - c0, c0, p.group_steps, u0, KIND == KIND_INT4, xsum, XR);
    __syncthreads();
    stream_steps<KIND, MT, NT, HZ, SD, 8>(q, p.M, wrow, ba, lds_x, lds_stride, a, b, c0, r, g, acc, accg);
  }
  if (KIND == KIND_INT8 && wv == 0) {  // the 128 offset over the whole range, once per workgroup
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const f32x4 xs = *reinterpret_cast<const f32x4*>(xsum + mt * 16 + g * 4);
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[t][mt][v] -= 128.f * xs[v];
    }
  }

  // ---- add the WK wavefronts' accumulators (LDS reuses the x staging area)
  constexpr int E = NT * MT * 256;  // accumulator values per wavefront
  __syncthreads();
  float* red = reinterpret_cast<float*>(lds_x);
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int v = 0; v < 4; ++v) red[wv * E + ((t * MT + mt) * 64 + lane) * 4 + v] = acc[t][mt][v];
  __syncthreads();

  const bool split = p.S > 1;
  for (int e = tid; e < E; e += blockDim.x) {
    const int v = e & 3, ln = (e >> 2) & 63, rest = e >> 8;
    const int mt = rest % MT, t = rest / MT;
    const int m = mt * 16 + (ln >> 4) * 4 + v;
    const int n = n0 + 16 * t + (ln & 15);
    if (m >= p.M || n >= p.N) continue;
    float o = 0.f;
    for (int w = 0; w < WK; ++w) o += red[w * E + e];
    if (split) {
      __hip_atomic_store(p.partial + ((int64_t)s * p.M + m) * p.N + n, o, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    } else {
      if (KIND == KIND_INT8)
        o = bf16_to_f32(f32_to_bf16(o)) * bf16_to_f32(f32_to_bf16(sd_to_f32<SD>(load_sd_raw<SD>(p.scale, n))));
      p.y[(int64_t)m * p.ldy + n] = f32_to_bf16(o);
    }
  }
  if (!split) return;

  // ---- split-K: the last workgroup of this row block adds the S partials in order
  __builtin_amdgcn_s_waitcnt(0);  // this thread's partial stores have completed
  __syncthreads();
  __shared__ int s_last;
  if (tid == 0)
    s_last = __hip_atomic_fetch_add(p.counters + blockIdx.x, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
             p.S - 1;
  __syncthreads();
  if (!s_last) return;
  for (int i = tid; i < p.M * rows; i += blockDim.x) {
    const int m = i / rows, n = n0 + (i - m * rows);
    if (n >= p.N) continue;
    float o = 0.f;
    for (int ss = 0; ss < p.S; ++ss)
      o += __hip_atomic_load(p.partial + ((int64_t)ss * p.M + m) * p.N + n, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
    if (KIND == KIND_INT8)
      o = bf16_to_f32(f32_to_bf16(o)) * bf16_to_f32(f32_to_bf16(sd_to_f32<SD>(load_sd_raw<SD>(p.scale, n))));
    p.y[(int64_t)m * p.ldy + n] = f32_to_bf16(o);
  }
  if (tid == 0) __hip_atomic_store(p.counters + blockIdx.x, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ------------------------------------------------------------------ host-side planning
struct Plan {
  int NT, WK, S, units, unit_steps, chunk_steps;
  size_t lds_bytes, counter_bytes, partial_bytes;
};

Plan make_plan(int64_t M, int64_t N, int64_t K, int weight_bits, int64_t group) {
  Plan pl;
  const int64_t steps = K / kStepK;
  pl.unit_steps = weight_bits == 4 ? (int)(group / kStepK) : 1;
  pl.units = (int)(steps / pl.unit_steps);
  const int MT = (int)((M + 15) / 16);
  // defaults: 16 rows per workgroup, 4 or 8 wavefronts on k slices, split K across
  // workgroups only while the row blocks alone cannot fill the GPU
  int NT = 1, WK = 8, S = 1;
  if (MT >= 2 && N % 32 == 0) NT = 2;
  if (MT >= 3) NT = 1;
  const int64_t tiles = (N + 16 * NT - 1) / (16 * NT);
  if (tiles >= 1024) WK = 4;
  int64_t want_blocks = 512;
  if (tiles < want_blocks) {
    int64_t sp = (want_blocks + tiles - 1) / tiles;
    const int64_t max_units_per_wave = 1;
    if (sp > pl.units / (WK * max_units_per_wave)) sp = pl.units / (WK * max_units_per_wave);
    S = (int)(sp < 1 ? 1 : sp);
  }
  const char* env = getenv("MIQ_WO_PLAN");
  if (env) {
    int a = 0, b = 0, c = 0;
    if (sscanf(env, "%d,%d,%d", &a, &b, &c) == 3 && (a == 1 || a == 2 || a == 4) && b >= 1 && b <= kMaxWaves && c >= 1) {
      NT = a;
      WK = b;
      S = c;
    }
  }
  if (MT * NT > 4) NT = 4 / MT;
  if (S > pl.units) S = pl.units;
  const int64_t nblk = (N + 16 * NT - 1) / (16 * NT);
  if (nblk > kMaxCounters) S = 1;
  pl.NT = NT;
  pl.WK = WK;
  pl.S = S;
  // x chunk in LDS: the split's whole range when it fits, else whole units that fit
  const int64_t split_steps = ((pl.units + S - 1) / S) * pl.unit_steps;
  int64_t cs = kLdsBudget / (M * kStepK * 2);
  cs = (cs / pl.unit_steps) * pl.unit_steps;
  if (cs < pl.unit_steps) cs = pl.unit_steps;
  if (cs > split_steps) cs = split_steps;
  pl.chunk_steps = (int)cs;
  const size_t red_bytes = (size_t)WK * NT * MT * 256 * 4;
  const size_t x_bytes = (size_t)M * (cs * kStepK + 8) * 2;
  // int4: scales and zeros of the workgroup's rows for the split's groups (<= 4 bytes each)
  // and the per-group activation sums; int8: one activation sum per row
  const int64_t ng_max = (pl.units + S - 1) / S;
  const size_t sz_bytes = (weight_bits == 4 ? (size_t)16 * NT * ng_max * 4 * 2 + (size_t)ng_max * 16 * MT * 4
                                            : (size_t)16 * MT * 4) + 16;
  pl.lds_bytes = x_bytes + sz_bytes > red_bytes ? x_bytes + sz_bytes : red_bytes;
  pl.counter_bytes = kMaxCounters * 4;
  pl.partial_bytes = S > 1 ? (size_t)S * M * N * 4 : 0;
  return pl;
}

template <int KIND, int MT, int NT, bool HZ, int SD>
void launch4(const WoParams& p, dim3 grid, int WK, size_t lds, hipStream_t st) {
  static bool attr = false;
  if (!attr) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&wo_gemm_kernel<KIND, MT, NT, HZ, SD>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, 80 * 1024);
    attr = true;
  }
  hipLaunchKernelGGL((wo_gemm_kernel<KIND, MT, NT, HZ, SD>), grid, dim3(64 * WK), lds, st, p);
}

template <int KIND, int MT, int NT, bool HZ>
void launch3(const WoParams& p, dim3 grid, int WK, size_t lds, hipStream_t st) {
  switch (p.sz_dtype) {
    case MIQ_BF16: launch4<KIND, MT, NT, HZ, MIQ_BF16>(p, grid, WK, lds, st); break;
    case MIQ_F16: launch4<KIND, MT, NT, HZ, MIQ_F16>(p, grid, WK, lds, st); break;
    default: launch4<KIND, MT, NT, HZ, MIQ_F32>(p, grid, WK, lds, st); break;
  }
}

template <int KIND, int MT, bool HZ>
void launch2(const WoParams& p, dim3 grid, int NT, int WK, size_t lds, hipStream_t st) {
  if (MT <= 2 && NT == 2) launch3<KIND, MT, (MT <= 2 ? 2 : 1), HZ>(p, grid, WK, lds, st);
  else launch3<KIND, MT, 1, HZ>(p, grid, WK, lds, st);
}

template <int KIND, bool HZ>
void launch(const WoParams& p, dim3 grid, int NT, int WK, size_t lds, hipStream_t st) {
  const int mt = (p.M + 15) / 16;
  switch (mt) {
    case 1: launch2<KIND, 1, HZ>(p, grid, NT, WK, lds, st); break;
    case 2: launch2<KIND, 2, HZ>(p, grid, NT, WK, lds, st); break;
    case 3: launch2<KIND, 3, HZ>(p, grid, NT, WK, lds, st); break;
    default: launch2<KIND, 4, HZ>(p, grid, NT, WK, lds, st); break;
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
  if (p.M <= 16 && !getenv("MIQ_WO_GENERAL")) {
    const int rc = wo_decode_launch(kind, p.x, p.ldx, p.w, p.ldw, p.scale, p.zero, p.sz_dtype, p.group_steps,
                                    p.ngroups, p.y, p.ldy, p.M, p.N, p.K, workspace, ws_bytes, kMaxCounters * 4, st);
    if (rc != -1) return rc;
  }
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
  const dim3 grid((unsigned)((p.N + 16 * pl.NT - 1) / (16 * pl.NT)), (unsigned)pl.S);
  if (kind == KIND_INT8) launch<KIND_INT8, false>(p, grid, pl.NT, pl.WK, pl.lds_bytes, st);
  else if (p.zero) launch<KIND_INT4, true>(p, grid, pl.NT, pl.WK, pl.lds_bytes, st);
  else launch<KIND_INT4, false>(p, grid, pl.NT, pl.WK, pl.lds_bytes, st);
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
