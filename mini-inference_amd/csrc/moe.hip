// INT4 mixture-of-experts decode layer for gfx950: moe_align + two grouped W4A16
// GEMMs (gate/up with the SiLU gate fused into its epilogue, then down with the
// routing weight) + a per-token combine in slot order.
//
// moe_align contract (as in the reference): the T*k (token, slot) pairs are grouped by
// expert, each group padded to a multiple of block_m with the sentinel T*k, expert_ids
// names the expert of each block_m-row tile (tiles past the end get E - 1), num_padded
// is the used length. Here the pairs inside a group are in ascending pair order: one
// wavefront per expert walks the pairs with ballots, so the layout is deterministic.
//
// The grouped GEMMs reuse the weight-only core (wo_core.h): a workgroup takes one
// 16-row tile of one expert, gathers its activation rows into LDS, and its four
// wavefronts stream 16 weight rows each.
#include "wo_core.h"

namespace miq {
namespace {

using namespace wo;

constexpr int kTile = 16;  // block_m: rows per tile

__device__ inline int load_id(const void* ids, int dtype, int i) {
  return dtype == MIQ_INT64 ? (int)static_cast<const int64_t*>(ids)[i] : static_cast<const int32_t*>(ids)[i];
}

__global__ void __launch_bounds__(1024)
moe_align_kernel(const void* __restrict__ ids, int dtype, int num_pairs, int E, int bm, int max_padded,
                 int max_blocks, int32_t* __restrict__ sorted_ids, int32_t* __restrict__ expert_ids,
                 int32_t* __restrict__ num_padded) {
  extern __shared__ int sm[];
  int* counts = sm;               // [E]
  int* offsets = sm + E;          // [E + 1]
  const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6), nw = blockDim.x >> 6;
  for (int e = tid; e < E; e += blockDim.x) counts[e] = 0;
  __syncthreads();
  for (int i = tid; i < num_pairs; i += blockDim.x) {
    const int e = load_id(ids, dtype, i);
    if (e >= 0 && e < E) atomicAdd(&counts[e], 1);
  }
  __syncthreads();
  if (tid == 0) {
    int total = 0;
    offsets[0] = 0;
    for (int e = 0; e < E; ++e) {
      total += (counts[e] + bm - 1) / bm * bm;
      offsets[e + 1] = total;
    }
    *num_padded = total;
  }
  __syncthreads();
  for (int i = tid; i < max_padded; i += blockDim.x) sorted_ids[i] = num_pairs;
  for (int t = tid; t < max_blocks; t += blockDim.x) {
    const int row = t * bm;
    int owner = E - 1;
    if (row < offsets[E]) {
      int lo = 0, hi = E - 1;
      while (lo < hi) {
        const int mid = (lo + hi) / 2;
        if (offsets[mid + 1] <= row) lo = mid + 1;
        else hi = mid;
      }
      owner = lo;
    }
    expert_ids[t] = owner;
  }
  __syncthreads();
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int e = wv; e < E; e += nw) {
    int base = offsets[e];
    for (int c0 = 0; c0 < num_pairs; c0 += 64) {
      const int i = c0 + lane;
      const bool hit = i < num_pairs && load_id(ids, dtype, i) == e;
      const uint64_t mask = __ballot(hit);
      if (hit) sorted_ids[base + __popcll(mask & below)] = i;
      base += __popcll(mask);
    }
  }
}

struct MoeParams {
  const uint16_t* hidden;
  int T, H, I, E, topk, num_pairs;
  const uint8_t* gu_q;
  const void* gu_s;
  const void* gu_z;
  const uint8_t* dn_q;
  const void* dn_s;
  const void* dn_z;
  int sz_dtype, group_steps;
  const uint16_t* topk_w;
  const int32_t* sorted_ids;
  const int32_t* expert_ids;
  const int32_t* num_padded;
  uint16_t* hbuf;  // [max_padded, I] bf16: silu(gate) * up per sorted row
  float* ypair;    // [num_pairs, H] fp32: routed down-projection per pair
  uint16_t* out;   // [T, H]
};

// Stage activation rows of a tile (row m -> source row src_row[m], < 0 = zero row),
// k-steps [kst0, kst0 + nsteps), into LDS in the int4 operand order.
__device__ inline void stage_rows(const uint16_t* base, int64_t ld, const int* src_row, uint16_t* lds,
                                  int lds_stride, int kst0, int nsteps) {
  const int pieces_per_row = nsteps * (kStepK / 8);
  for (int i = threadIdx.x; i < kTile * pieces_per_row; i += 256) {
    const int m = i / pieces_per_row, c = i - m * pieces_per_row;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (src_row[m] >= 0)
      v = permute_for_u4(*reinterpret_cast<const uint4*>(base + src_row[m] * ld + (int64_t)kst0 * kStepK + c * 8));
    *reinterpret_cast<uint4*>(lds + m * lds_stride + c * 8) = v;
  }
}

__device__ inline float bf16r(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// Stream all k-steps of one 16-row weight tile (row `row` of lane r) against the
// staged activation rows; returns the tile's 16x16 result in C layout.
template <bool HZ, int SD>
__device__ inline f32x4 tile_product(const MoeParams& p, const uint8_t* wbase, int64_t row, int K,
                                     const void* sc, const void* zr, const uint16_t* src, int64_t ld,
                                     const int* src_row, uint16_t* lds, int chunk_steps, int r, int g,
                                     const int64_t (&tile_rows)[4], int wv) {
  const uint8_t* wrow[1] = {wbase + row * (K / 2)};
  f32x4 acc[1][1], accg[1][1];
  const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
  acc[0][0] = z4;
  accg[0][0] = z4;
  const int lds_stride = chunk_steps * kStepK + 8;
  const int steps = K / kStepK;
  const int ngroups = steps / p.group_steps;
  // LDS: [activation chunk][activation sums per group][scales of the 4 wavefronts'
  // 16-row tiles][zeros]
  float* xsum = reinterpret_cast<float*>(lds + kTile * lds_stride);
  typedef typename GroupQ<SD>::raw_t raw_t;
  raw_t* lsc = reinterpret_cast<raw_t*>(xsum + ngroups * kTile);
  raw_t* lzr = lsc + 64 * ngroups;
  const GroupQ<SD> q{lsc + wv * 16 * ngroups, HZ ? lzr + wv * 16 * ngroups : nullptr, ngroups, 0, p.group_steps,
                     xsum, kTile};
  for (int i = threadIdx.x; i < ngroups * kTile; i += blockDim.x) xsum[i] = 0.f;
  for (int c0 = 0; c0 < steps; c0 += chunk_steps) {
    const int c1 = min(steps, c0 + chunk_steps);
    Batch<KIND_INT4, 1, 16> bt;
    load_batch<KIND_INT4, 1, 16>(wrow, bt, c0, c1, g);  // in flight during staging
    if (c0) __syncthreads();
    stage_rows(src, ld, src_row, lds, lds_stride, c0, c1 - c0);
    if (c0 == 0) {
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        stage_groups<SD>(sc, ngroups, tile_rows[w], 16, 0, ngroups, lsc + w * 16 * ngroups);
        if (HZ) stage_groups<SD>(zr, ngroups, tile_rows[w], 16, 0, ngroups, lzr + w * 16 * ngroups);
      }
    }
    __syncthreads();
    sum_activations(lds, lds_stride, kTile, c1 - c0, c0, p.group_steps, 0, true, xsum, kTile);
    __syncthreads();
    stream_steps<KIND_INT4, 1, 1, HZ, SD, 16>(q, kTile, wrow, bt, lds, lds_stride, c0, c1, c0, r, g, acc, accg);
  }
  return acc[0][0];
}

// gate/up: workgroup = (32 columns of I, one tile); waves 0-1 gate rows, 2-3 up rows
template <bool HZ, int SD>
__global__ void __launch_bounds__(256)
moe_gate_up_kernel(MoeParams p, int chunk_steps) {
  extern __shared__ __align__(16) uint16_t lds[];
  __shared__ int s_src[kTile];
  __shared__ float s_gu[4][kTile][16 + 1];
  const int tile = blockIdx.y;
  if (tile * kTile >= *p.num_padded) return;
  const int e = p.expert_ids[tile];
  const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6), r = lane & 15, g = lane >> 4;
  if (tid < kTile) {
    const int pair = p.sorted_ids[tile * kTile + tid];
    s_src[tid] = pair < p.num_pairs ? pair / p.topk : -1;
  }
  __syncthreads();
  const int n0 = blockIdx.x * 32;
  const int64_t base = (int64_t)e * 2 * p.I + n0;
  const int64_t tile_rows[4] = {base, base + 16, base + p.I, base + p.I + 16};
  const int64_t row = tile_rows[wv] + r;
  const f32x4 acc = tile_product<HZ, SD>(p, p.gu_q, row, p.H, p.gu_s, p.gu_z, p.hidden, p.H, s_src, lds,
                                         chunk_steps, r, g, tile_rows, wv);
#pragma unroll
  for (int v = 0; v < 4; ++v) s_gu[wv][g * 4 + v][r] = acc[v];
  __syncthreads();
  // h[m][c] = silu(gate) * up with the reference's bf16 roundings, c in [0, 32)
  for (int i = tid; i < kTile * 32; i += 256) {
    const int m = i >> 5, c = i & 31;
    const float gt = bf16r(s_gu[(c >> 4)][m][c & 15]);
    const float up = bf16r(s_gu[2 + (c >> 4)][m][c & 15]);
    const float act = bf16r(gt / (1.f + __expf(-gt)));
    p.hbuf[(int64_t)(tile * kTile + m) * p.I + n0 + c] = f32_to_bf16(act * up);
  }
}

// down: workgroup = (64 columns of H, one tile)
template <bool HZ, int SD>
__global__ void __launch_bounds__(256)
moe_down_kernel(MoeParams p, int chunk_steps) {
  extern __shared__ __align__(16) uint16_t lds[];
  __shared__ int s_src[kTile];
  const int tile = blockIdx.y;
  if (tile * kTile >= *p.num_padded) return;
  const int e = p.expert_ids[tile];
  const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6), r = lane & 15, g = lane >> 4;
  if (tid < kTile) {
    const int pair = p.sorted_ids[tile * kTile + tid];
    s_src[tid] = pair < p.num_pairs ? tile * kTile + tid : -1;
  }
  __syncthreads();
  const int n = blockIdx.x * 64 + wv * 16 + r;
  const int64_t base = (int64_t)e * p.H + blockIdx.x * 64;
  const int64_t tile_rows[4] = {base, base + 16, base + 32, base + 48};
  const int64_t row = base + wv * 16 + r;
  const f32x4 acc = tile_product<HZ, SD>(p, p.dn_q, row, p.I, p.dn_s, p.dn_z, p.hbuf, p.I, s_src, lds,
                                         chunk_steps, r, g, tile_rows, wv);
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int m = g * 4 + v;
    const int pair = p.sorted_ids[tile * kTile + m];
    if (pair < p.num_pairs) {
      const float w = bf16_to_f32(p.topk_w[pair]);
      p.ypair[(int64_t)pair * p.H + n] = bf16r(bf16r(acc[v]) * w);
    }
  }
}

// out[t][n] = sum over slots j (in order) of ypair[t * k + j][n]
__global__ void moe_combine_kernel(const float* __restrict__ ypair, int topk, int H, uint16_t* __restrict__ out) {
  const int t = blockIdx.y;
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= H) return;
  float s = 0.f;
  for (int j = 0; j < topk; ++j) s += ypair[((int64_t)t * topk + j) * H + n];
  out[(int64_t)t * H + n] = f32_to_bf16(s);
}

template <bool HZ, int SD>
void launch_experts_t(const MoeParams& p, dim3 gu_grid, dim3 dn_grid, int gu_chunk, int dn_chunk, size_t gu_lds,
                      size_t dn_lds, hipStream_t st) {
  hipLaunchKernelGGL((moe_gate_up_kernel<HZ, SD>), gu_grid, dim3(256), gu_lds, st, p, gu_chunk);
  hipLaunchKernelGGL((moe_down_kernel<HZ, SD>), dn_grid, dim3(256), dn_lds, st, p, dn_chunk);
}

void launch_experts(const MoeParams& p, bool hz, int sd, dim3 gu_grid, dim3 dn_grid, int gu_chunk, int dn_chunk,
                    size_t gu_lds, size_t dn_lds, hipStream_t st) {
#define MIQ_EXPERTS(HZV, SDV) launch_experts_t<HZV, SDV>(p, gu_grid, dn_grid, gu_chunk, dn_chunk, gu_lds, dn_lds, st)
  if (hz) {
    if (sd == MIQ_BF16) MIQ_EXPERTS(true, MIQ_BF16);
    else if (sd == MIQ_F16) MIQ_EXPERTS(true, MIQ_F16);
    else MIQ_EXPERTS(true, MIQ_F32);
  } else {
    if (sd == MIQ_BF16) MIQ_EXPERTS(false, MIQ_BF16);
    else if (sd == MIQ_F16) MIQ_EXPERTS(false, MIQ_F16);
    else MIQ_EXPERTS(false, MIQ_F32);
  }
#undef MIQ_EXPERTS
}

size_t max_padded_rows(int64_t num_pairs, int64_t E) { return (size_t)(num_pairs + E * (kTile - 1)); }

}  // namespace
}  // namespace miq

using namespace miq;

extern "C" int miq_moe_align(const void* topk_ids, int idx_dtype, int64_t num_pairs, int64_t E, int64_t block_m,
                             int32_t* sorted_ids, int32_t* expert_ids, int32_t* num_padded, void* stream) {
  MIQ_REQUIRE(idx_dtype == MIQ_INT32 || idx_dtype == MIQ_INT64, "moe_align: topk_ids must be int32 or int64");
  MIQ_REQUIRE(num_pairs >= 1 && num_pairs < (1LL << 30) && E >= 1 && E <= 4096 && block_m >= 1 &&
                  block_m <= 1024,
              "moe_align: bad sizes pairs=%lld E=%lld block_m=%lld", (long long)num_pairs, (long long)E,
              (long long)block_m);
  const int64_t max_padded = num_pairs + E * (block_m - 1);
  const int64_t max_blocks = (max_padded + block_m - 1) / block_m;
  hipLaunchKernelGGL(moe_align_kernel, dim3(1), dim3(1024), (size_t)(2 * E + 1) * sizeof(int),
                     (hipStream_t)stream, topk_ids, idx_dtype, (int)num_pairs, (int)E, (int)block_m,
                     (int)max_padded, (int)max_blocks, sorted_ids, expert_ids, num_padded);
  return check_launch("moe_align");
}

extern "C" size_t miq_moe_workspace_bytes(int64_t T, int64_t topk, int64_t E, int64_t H, int64_t I) {
  const size_t hb = max_padded_rows(T * topk, E) * (size_t)I * 2;
  return ((hb + 255) / 256) * 256 + (size_t)T * topk * H * 4;
}

extern "C" int miq_w4a16_moe(const void* hidden, int64_t T, int64_t H, int64_t I, int64_t E, int64_t topk,
                             const uint8_t* gu_q, const void* gu_scale, const void* gu_zero,
                             const uint8_t* dn_q, const void* dn_scale, const void* dn_zero,
                             int sz_dtype, int64_t group, const void* topk_weights,
                             const int32_t* sorted_ids, const int32_t* expert_ids,
                             const int32_t* num_padded, void* workspace, size_t workspace_bytes,
                             void* out, void* stream) {
  MIQ_REQUIRE(sz_dtype == MIQ_F32 || sz_dtype == MIQ_BF16 || sz_dtype == MIQ_F16, "w4a16_moe: bad scale dtype");
  MIQ_REQUIRE(group >= kStepK && group % kStepK == 0 && H % group == 0 && I % group == 0,
              "w4a16_moe: group=%lld must be a multiple of 128 dividing H and I", (long long)group);
  MIQ_REQUIRE(H % 64 == 0 && I % 32 == 0 && T >= 1 && topk >= 1 && E >= 1 && H < (1 << 20) && I < (1 << 20),
              "w4a16_moe: H must be a multiple of 64 and I of 32");
  MIQ_REQUIRE((gu_zero == nullptr) == (dn_zero == nullptr), "w4a16_moe: zero points for both or neither");
  MIQ_REQUIRE(((reinterpret_cast<uintptr_t>(hidden) | reinterpret_cast<uintptr_t>(gu_q) |
                reinterpret_cast<uintptr_t>(dn_q)) & 15) == 0,
              "w4a16_moe: hidden and weights must be 16-byte aligned");
  const size_t need = miq_moe_workspace_bytes(T, topk, E, H, I);
  MIQ_REQUIRE(workspace != nullptr && workspace_bytes >= need, "w4a16_moe: workspace of %zu bytes needed", need);
  MoeParams p{};
  p.hidden = static_cast<const uint16_t*>(hidden);
  p.T = (int)T;
  p.H = (int)H;
  p.I = (int)I;
  p.E = (int)E;
  p.topk = (int)topk;
  p.num_pairs = (int)(T * topk);
  p.gu_q = gu_q;
  p.gu_s = gu_scale;
  p.gu_z = gu_zero;
  p.dn_q = dn_q;
  p.dn_s = dn_scale;
  p.dn_z = dn_zero;
  p.sz_dtype = sz_dtype;
  p.group_steps = (int)(group / kStepK);
  p.topk_w = static_cast<const uint16_t*>(topk_weights);
  p.sorted_ids = sorted_ids;
  p.expert_ids = expert_ids;
  p.num_padded = num_padded;
  const size_t max_rows = max_padded_rows(T * topk, E);
  const size_t hb = ((max_rows * I * 2 + 255) / 256) * 256;
  p.hbuf = static_cast<uint16_t*>(workspace);
  p.ypair = reinterpret_cast<float*>(static_cast<char*>(workspace) + hb);
  p.out = static_cast<uint16_t*>(out);
  const unsigned tiles = (unsigned)((max_rows + kTile - 1) / kTile);
  hipStream_t st = (hipStream_t)stream;
  // LDS chunk: 16 rows x up to 1024 k (32 KiB)
  const int gu_chunk = (int)std::min<int64_t>(8, H / kStepK);
  const int dn_chunk = (int)std::min<int64_t>(8, I / kStepK);
  const size_t gu_lds = (size_t)kTile * (gu_chunk * kStepK + 8) * 2 + (size_t)64 * (H / group) * 4 * 2 +
                        (size_t)kTile * (H / group) * 4;
  const size_t dn_lds = (size_t)kTile * (dn_chunk * kStepK + 8) * 2 + (size_t)64 * (I / group) * 4 * 2 +
                        (size_t)kTile * (I / group) * 4;
  const dim3 gu_grid((unsigned)(I / 32), tiles), dn_grid((unsigned)(H / 64), tiles);
  launch_experts(p, gu_zero != nullptr, sz_dtype, gu_grid, dn_grid, gu_chunk, dn_chunk, gu_lds, dn_lds, st);
  int rc = check_launch("w4a16_moe experts");
  if (rc) return rc;
  hipLaunchKernelGGL(moe_combine_kernel, dim3((unsigned)((H + 255) / 256), (unsigned)T), dim3(256), 0, st,
                     p.ypair, (int)topk, (int)H, p.out);
  return check_launch("w4a16_moe combine");
}
